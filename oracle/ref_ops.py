"""torch-CPU fp32 restatement of ``reference/ref_ops.py`` (test infrastructure, see ``oracle/__init__``).

Every function returns new tensors (the reference's functional style, reference/ref_ops.py:1-4) and rounds to fp16
at the same points as the reference:
  * ``gemv_ref``                  fp32 matvec of the fp16 (dequantized) weight, fp16 out        ref_ops.py:10-12
  * ``add_rmsnorm_ref``           fp16 residual add; fp32 mean-square; fp16(x*rsqrt); fp16 w*h   ref_ops.py:15-20
  * ``swiglu_ref``                fp16(silu(fp32 gate)) times up, fp16 product                   ref_ops.py:23-27
  * ``rope_tables``               float64 angles pos * theta^(-2i/D) -> float32 cos/sin          ref_ops.py:30-33
  * ``rope_ref``                  rotate_half pairs (i, i+D/2), fp32 math, fp16 out              ref_ops.py:36-41
  * ``rope_append_ref``           RoPE on q,k and paged K/V append at ``pos``                    ref_ops.py:44-53
  * ``gather_kv``                 paged [pages, n_kv, P, D] -> contiguous [ctx, n_kv, D]         ref_ops.py:56-62
  * ``attention_contiguous_ref``  GQA softmax(q k^T / sqrt(D)) v, fp32, fp16 out                 ref_ops.py:65-73
  * ``paged_attention_ref``       gather + attention                                             ref_ops.py:76-78
  * ``split_softmax_combine_ref`` split-K partials (o, m, l) + log-sum-exp combine               ref_ops.py:81-96
"""
import math

import torch

F32 = torch.float32
F16 = torch.float16


def gemv_ref(w_ref: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """y[N] = fp16(sum_k float(W[n,k]) * float(x[k])), fp32 accumulation (ref_ops.py:10-12)."""
    return torch.mv(w_ref.to(F32), x.reshape(-1).to(F32)).to(F16)


def add_rmsnorm_ref(x: torch.Tensor, delta, w: torch.Tensor, eps: float):
    """Returns (x_new, out): x_new = x + delta in fp16 (x itself if delta is None);
    out = w * fp16(float(x_new) * rsqrt(mean(float(x_new)^2) + eps)) (ref_ops.py:15-20)."""
    x_new = x if delta is None else torch.add(x, delta)
    xf = x_new.to(F32)
    inv = torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)
    return x_new, torch.mul(w, (xf * inv).to(F16))


def swiglu_ref(gu: torch.Tensor) -> torch.Tensor:
    """gu = [gate | up] -> fp16(silu(float(gate))) * up with one fp16 rounding of the product (ref_ops.py:23-27)."""
    inter = gu.shape[-1] // 2
    gate, up = gu[..., :inter], gu[..., inter:]
    s16 = torch.nn.functional.silu(gate.to(F32)).to(F16)
    return (s16.to(F32) * up.to(F32)).to(F16)


def rope_tables(max_pos: int, head_dim: int = 64, theta: float = 10000.0, device="cpu"):
    """(cos, sin) float32 [max_pos, head_dim/2]; angle(p, i) = p * theta^(-2i/head_dim) in float64 (ref_ops.py:30-33)."""
    i2 = torch.arange(0, head_dim, 2, dtype=torch.float64, device=device)
    inv_freq = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64, device=device), i2 / head_dim)
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float64, device=device), inv_freq)
    return torch.cos(ang).to(F32).contiguous(), torch.sin(ang).to(F32).contiguous()


def rope_ref(x: torch.Tensor, cos, sin, pos: int) -> torch.Tensor:
    """x [heads, D]; rotate pairs (i, i+D/2): (a c - b s, b c + a s) in fp32, fp16 out (ref_ops.py:36-41)."""
    half = x.shape[-1] // 2
    a = x[..., :half].to(F32)
    b = x[..., half:].to(F32)
    c, s = cos[pos], sin[pos]
    lo = a * c - b * s
    hi = b * c + a * s
    return torch.cat([lo, hi], dim=-1).to(F16)


def rope_append_ref(qkv, cos, sin, pos, k_cache, v_cache, block_table, n_q, n_kv, D, page):
    """Rotate q and k at position ``pos``, write k (rotated) and v (copied) to physical page block_table[pos // page],
    slot pos % page of the caches (modified in place). Returns the rotated q [n_q, D] (ref_ops.py:44-53)."""
    q = qkv[: n_q * D].reshape(n_q, D)
    k = qkv[n_q * D:(n_q + n_kv) * D].reshape(n_kv, D)
    v = qkv[(n_q + n_kv) * D:(n_q + 2 * n_kv) * D].reshape(n_kv, D)
    q_rot = rope_ref(q, cos, sin, pos)
    k_rot = rope_ref(k, cos, sin, pos)
    phys = int(block_table[pos // page])
    slot = pos % page
    k_cache[phys, :, slot, :] = k_rot
    v_cache[phys, :, slot, :] = v
    return q_rot


def gather_kv(k_cache, v_cache, block_table, ctx, page):
    """Paged caches [pages, n_kv, P, D] -> contiguous K, V [ctx, n_kv, D]; token t lives in physical page
    block_table[t // P] at slot t % P (ref_ops.py:56-62)."""
    t = torch.arange(ctx)
    phys = block_table.to(torch.long)[t // page]
    slot = t % page
    return k_cache[phys, :, slot, :], v_cache[phys, :, slot, :]


def _kv_head_of(n_q, n_kv):
    """query head h reads kv head h // (n_q / n_kv) (repeat_interleave grouping, ref_ops.py:68-70)."""
    return torch.arange(n_q) // (n_q // n_kv)


def attention_contiguous_ref(q, k, v):
    """q [n_q, D], k/v [ctx, n_kv, D] -> fp16 [n_q, D]; fp32 scores / sqrt(D), fp32 softmax (ref_ops.py:65-73)."""
    n_q, D = q.shape
    kvh = _kv_head_of(n_q, k.shape[1])
    kf = k.to(F32)[:, kvh, :].permute(1, 0, 2)            # [n_q, ctx, D]
    vf = v.to(F32)[:, kvh, :].permute(1, 0, 2)
    scores = torch.bmm(kf, q.to(F32).unsqueeze(-1)).squeeze(-1) / math.sqrt(D)   # [n_q, ctx]
    p = torch.softmax(scores, dim=-1)
    return torch.bmm(p.unsqueeze(1), vf).squeeze(1).to(F16)


def paged_attention_ref(q, k_cache, v_cache, block_table, ctx, page):
    """gather_kv then attention_contiguous_ref (ref_ops.py:76-78)."""
    k, v = gather_kv(k_cache, v_cache, block_table, ctx, page)
    return attention_contiguous_ref(q, k, v)


def split_partials_ref(q, k, v, part):
    """Per-split unnormalized (o [S, n_q, D], m [S, n_q], l [S, n_q]) over token ranges [s*part, (s+1)*part)
    (the partial half of ref_ops.py:81-91)."""
    n_q, D = q.shape
    kvh = _kv_head_of(n_q, k.shape[1])
    kf = k.to(F32)[:, kvh, :].permute(1, 0, 2)
    vf = v.to(F32)[:, kvh, :].permute(1, 0, 2)
    qf = q.to(F32).unsqueeze(-1)
    os_, ms, ls = [], [], []
    for t0 in range(0, k.shape[0], part):
        sc = torch.bmm(kf[:, t0:t0 + part], qf).squeeze(-1) / math.sqrt(D)
        m = sc.max(dim=-1).values
        p = torch.exp(sc - m[:, None])
        os_.append(torch.bmm(p.unsqueeze(1), vf[:, t0:t0 + part]).squeeze(1))
        ms.append(m)
        ls.append(p.sum(dim=-1))
    return torch.stack(os_), torch.stack(ms), torch.stack(ls)


def combine_ref(o, m, l):
    """Log-sum-exp combine of split partials: M = max_s m_s; O = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s
    (ref_ops.py:92-96). Returns fp16 [n_q, D]."""
    M = m.max(dim=0).values
    a = torch.exp(m - M)
    L = (a * l).sum(dim=0)
    return ((a[..., None] * o).sum(dim=0) / L[:, None]).to(F16)


def split_softmax_combine_ref(q, k, v, part):
    """Pure-CPU model of the split-K kernel: partials then combine (ref_ops.py:81-96)."""
    return combine_ref(*split_partials_ref(q, k, v, part))
