"""INT4 weight format for the W4A16 GEMV, and its producers.

Same format and same numbers as the reference's ``runtime/quant.py``: weight W [N, K] -> ``packed`` int32 [N, K/8]
(word j holds elements 8j..8j+7; element 8j+2i at bits [4i, 4i+4), element 8j+2i+1 at bits [16+4i, 20+4i)) and
``sz`` fp16 [N, K/G, 2] = (scale, zero) per (row, group), with scale = fp16((max - min) / 15) (floored at 1e-6),
zero = rint(-min / scale) in [0, 15], q = clamp(rint(w / scale) + zero, 0, 15).

Producers:
  * RTN and range-clipped RTN (``quantize_pack(w, group, clip)``): one HIP kernel (dk_quantize_w4) quantizes and
    packs on the GPU, so building a Llama-3-8B-sized model does not round-trip 16 GB of weights through the host.
  * GPTQ (``quantize_gptq``, runtime/quant.py:51-90 of the reference): the column-by-column error feedback through
    the inverse input Hessian, in torch on whatever device the weight lives on (a calibration-time algorithm built
    from Cholesky factorizations and small GEMMs, not a decode kernel), then ``pack_codes`` to the same format.
    ``runtime.gptq.calibrate`` produces the Hessians from calibration tokens.
"""
import torch

from . import ext

# runtime/quant.py:17 of the reference: range factors tried per group by the clipping search
CLIP_GRID = (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7)


def quantize_pack(w: torch.Tensor, group: int, clip: bool = False):
    """fp16 CUDA tensor [N, K] -> (packed int32 [N, K/8], sz fp16 [N, K/G, 2]) on the same device (RTN, or
    range-clipped RTN with clip=True)."""
    if not w.is_cuda:
        raise RuntimeError("quantize_pack: w must be a CUDA tensor (the format is produced by the HIP kernel)")
    N, K = w.shape
    if K % group:
        raise RuntimeError(f"K={K} is not a multiple of group={group}")
    w16 = w.to(torch.float16).contiguous()
    packed = torch.empty(N, K // 8, dtype=torch.int32, device=w.device)
    sz = torch.empty(N, K // group, 2, dtype=torch.float16, device=w.device)
    ext.load().quantize_w4(w16, packed, sz, group, clip)
    return packed, sz


def group_params(wf: torch.Tensor, clip: bool = False):
    """wf fp32 [..., G] -> (scale, zero) fp32 [..., 1]: the parameters of each group of G weights (the convention of
    runtime/quant.py:20-38 of the reference): scale = fp16((hi - lo) / 15) floored at 1e-6 and read back as fp32,
    zero = rint(-lo / scale) clamped to [0, 15].

    Without clip, [lo, hi] is the group's range. With clip, every factor a of CLIP_GRID shrinks it to [a lo, a hi];
    the candidates are evaluated together along a leading grid axis and each group keeps the factor with the
    smallest sum of squared rounding errors (fp32 terms, summed over the group in fp32), the first one on ties
    (argmin's choice, the same as a strict-less-than scan over the grid in order)."""
    lo, hi = wf.amin(-1, keepdim=True), wf.amax(-1, keepdim=True)

    def params(a_lo, a_hi):
        scale = ((a_hi - a_lo) / 15).clamp(min=1e-6).half().float()
        return scale, torch.round(-a_lo / scale).clamp(0, 15)

    if not clip:
        return params(lo, hi)
    a = torch.tensor(CLIP_GRID, dtype=wf.dtype, device=wf.device).view(-1, *([1] * wf.dim()))
    scale, zero = params(lo.unsqueeze(0) * a, hi.unsqueeze(0) * a)                  # [F, ..., 1]
    wq = torch.clamp(torch.round(wf.unsqueeze(0) / scale) + zero, 0, 15)
    err = ((wq - zero) * scale - wf.unsqueeze(0)).pow(2).sum(-1, keepdim=True)       # [F, ..., 1]
    pick = err.argmin(dim=0, keepdim=True)
    return scale.gather(0, pick).squeeze(0), zero.gather(0, pick).squeeze(0)


class _InverseHessianFactor:
    """U = the upper Cholesky factor of (H + damp * mean(diag H) * I)^-1, the quantity GPTQ propagates rounding errors
    through (Frantar et al. 2022, section 3.3: row j of U holds the error weights of column j onto columns >= j).
    Input channels that never fire (H_jj = 0) are given H_jj = 1 before damping; their weights are zeroed by the
    caller, so they quantize to the zero point and spread no error."""

    def __init__(self, H: torch.Tensor, damp: float):
        H = H.float().clone()
        self.dead = torch.diag(H) == 0
        H[self.dead, self.dead] = 1
        H += damp * torch.diag(H).mean() * torch.eye(H.shape[0], device=H.device)
        chol = torch.linalg.cholesky(H)                       # H = L L^T
        self.U = torch.linalg.cholesky(torch.cholesky_inverse(chol), upper=True)


@torch.no_grad()
def quantize_gptq(w: torch.Tensor, H: torch.Tensor, group: int, clip: bool = False, damp: float = 0.01,
                  block: int = 128):
    """GPTQ (Frantar et al. 2022, Algorithm 1) into the format of ``quantize``: returns (q uint8 [N, K], scale,
    zero fp16 [N, K/G]), with the numbers of runtime/quant.py:51-90 of the reference.

    The weight is swept left to right in blocks of ``block`` columns, in place on an fp32 copy:
      * when a column starts a group, the group's (scale, zero) come from its columns as they stand then, i.e.
        after the errors of every earlier column were spread onto them (``group_params``; no activation
        reordering, so groups stay contiguous and the GEMV reads the result unchanged);
      * column j is rounded with its group's parameters; its error e = (w_j - deq(q_j)) / U_jj is subtracted,
        weighted by row j of U, from the columns j .. end of the block (a rank-1 update);
      * at the end of a block, the block's errors reach every later column at once through one GEMM with the
        U rows of the block ("lazy batch update").
    The layer output error ||X W^T - X deq(Q)^T|| (H = 2 X^T X / n) is minimised rather than the weight error."""
    N, K = w.shape
    if K % group or block % group:
        raise ValueError(f"K={K} and block={block} must be multiples of group={group}")
    hf = _InverseHessianFactor(H, damp)
    U = hf.U
    W = w.float().clone()
    W[:, hf.dead] = 0
    codes = torch.zeros(N, K, dtype=torch.uint8, device=W.device)
    scales = torch.zeros(N, K // group, device=W.device)
    zeros = torch.zeros(N, K // group, device=W.device)
    for b0 in range(0, K, block):
        b1 = min(b0 + block, K)
        errs = torch.zeros(N, b1 - b0, device=W.device)
        for j in range(b0, b1):
            if j % group == 0:                                   # block % group == 0: the group lies in this block
                s, z = group_params(W[:, j:j + group], clip)
                scales[:, j // group], zeros[:, j // group] = s[:, 0], z[:, 0]
            g = j // group
            sc, zp = scales[:, g], zeros[:, g]
            col = W[:, j]
            qj = torch.clamp(torch.round(col / sc) + zp, 0, 15)
            codes[:, j] = qj.to(torch.uint8)
            e = (col - (qj - zp) * sc) / U[j, j]
            W[:, j:b1] -= e[:, None] * U[j, j:b1][None, :]
            errs[:, j - b0] = e
        W[:, b1:] -= errs @ U[b0:b1, b1:]
    return codes, scales.half(), zeros.half()


def pack_codes(q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor):
    """Codes uint8 [N, K] and fp16 scale / zero [N, K/G] -> (packed int32 [N, K/8], sz fp16 [N, K/G, 2]) on q's
    device (runtime/quant.py:100-109 pack, :122-124 pack_scale_zero)."""
    N, K = q.shape
    c = q.to(torch.int64).view(N, K // 8, 8)
    word = torch.zeros(N, K // 8, dtype=torch.int64, device=q.device)
    for e in range(8):
        word |= c[..., e] << (4 * (e >> 1) + 16 * (e & 1))
    packed = torch.where(word >= 1 << 31, word - (1 << 32), word).to(torch.int32)
    sz = torch.stack([scale.half(), zero.half()], dim=-1).contiguous()
    return packed, sz


class QuantLinear:
    """One quantized weight in kernel format (runtime/quant.py:127-140): RTN or range-clipped RTN by the HIP producer,
    or precomputed codes ``qsz = (q, scale, zero)`` (e.g. from ``runtime.gptq.calibrate``) packed on the device."""

    def __init__(self, w: torch.Tensor, group: int, keep_ref: bool = False, clip: bool = False, qsz=None):
        if keep_ref:
            raise NotImplementedError("the dequantized fp16 reference weight belongs to the CPU oracle, not here")
        self.N, self.K = w.shape
        self.group = group
        if qsz is not None:
            q, s, z = (t.to(w.device) for t in qsz)
            if q.shape != (self.N, self.K) or s.shape != (self.N, self.K // group) or z.shape != s.shape:
                raise ValueError(f"precomputed codes {tuple(q.shape)} / {tuple(s.shape)} do not fit W {tuple(w.shape)}"
                                 f" at group {group}")
            self.packed, self.sz = pack_codes(q, s, z)
        else:
            self.packed, self.sz = quantize_pack(w, group, clip)
        self.w_ref = None

    def nbytes(self):
        return self.packed.numel() * 4 + self.sz.numel() * 2
