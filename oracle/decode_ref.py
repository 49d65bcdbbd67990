"""CPU decode step of the reference runtime with ``backend="ref"`` (test infrastructure, see ``oracle/__init__``).

Restates the composition of ``runtime/model.py:216-233`` (one token) using only ``oracle.ref_ops``:

    x = emb[tok]
    per layer:  add_norm(delta, ln1) -> qkv GEMV -> rope_append + paged attention at ctx = pos + 1 -> o GEMV
                -> add_norm(o, ln2) -> gate|up GEMV -> SwiGLU -> down GEMV;  delta = down
    add_norm(delta, norm_f) -> LM-head GEMV -> argmax -> pos + 1

``add_norm`` writes the residual sum back into x only when a delta is given (runtime/model.py:189-196); the first
layer therefore normalises the embedding row itself. Weights are the fp16 dequantized ``w_ref`` of each fused
projection (qkv = cat(q, k, v), gu = cat(gate, up), runtime/model.py:98-106). The KV cache is
[L, 2, pages, n_kv, P, D] fp16 with one block table shared by all layers (runtime/model.py:117-120).

``steps`` runs T consecutive steps at once (teacher forcing: each row's input token is given): the same ops with the
same rounding points applied to every row, the projections as one fp32 matrix product, each row attending the cache
up to its own position. It is the same function as T calls of ``step`` up to the fp32 summation order of the products
(pinned against ``step`` in tests/test_oracle.py), and costs one pass over the weights instead of T.
"""
import math

import torch

from . import ref_ops as R


class RefDecoder:
    def __init__(self, weights, shape, max_ctx, page, block_table, rope_theta=10000.0):
        """weights: {"emb" [V,H], "norm_f" [H], "lm_head" [V,H], "layers": [{"ln1","ln2","qkv","o","gu","down"}]}
        (all fp16 CPU tensors, projections already dequantized); shape: object with hidden_size,
        num_hidden_layers, num_attention_heads, num_key_value_heads, intermediate_size, vocab_size, rms_norm_eps."""
        self.w = weights
        self.H = shape.hidden_size
        self.L = shape.num_hidden_layers
        self.n_q = shape.num_attention_heads
        self.n_kv = shape.num_key_value_heads
        self.D = self.H // self.n_q
        self.eps = shape.rms_norm_eps
        self.page = page
        self.bt = block_table.to(torch.int32).cpu()
        n_pages = int(self.bt.numel())
        self.kv = torch.zeros(self.L, 2, n_pages, self.n_kv, page, self.D, dtype=torch.float16)
        self.cos, self.sin = R.rope_tables(max_ctx + 1, self.D, rope_theta)

    def step(self, tok: int, pos: int):
        """One decode step at position ``pos`` for input token ``tok``; returns (logits fp16 [V], argmax token)."""
        w = self.w
        x = w["emb"][tok].clone()
        delta = None
        for li, lw in enumerate(w["layers"]):
            x, normed = R.add_rmsnorm_ref(x, delta, lw["ln1"], self.eps)
            qkv = R.gemv_ref(lw["qkv"], normed)
            kc, vc = self.kv[li, 0], self.kv[li, 1]
            q = R.rope_append_ref(qkv, self.cos, self.sin, pos, kc, vc, self.bt, self.n_q, self.n_kv, self.D,
                                  self.page)
            attn = R.paged_attention_ref(q, kc, vc, self.bt, pos + 1, self.page)
            o = R.gemv_ref(lw["o"], attn.reshape(-1))
            x, normed = R.add_rmsnorm_ref(x, o, lw["ln2"], self.eps)
            gu = R.gemv_ref(lw["gu"], normed)
            act = R.swiglu_ref(gu)
            delta = R.gemv_ref(lw["down"], act)
        x, normed = R.add_rmsnorm_ref(x, delta, w["norm_f"], self.eps)
        logits = R.gemv_ref(w["lm_head"], normed)
        return logits, int(torch.argmax(logits.to(torch.float32)))

    def steps(self, tokens, pos0: int):
        """Steps for input tokens[t] at positions pos0 + t, t < T, in one batched pass (K/V rows of every position
        written to the cache, row t attending positions 0 .. pos0 + t); returns (logits fp16 [T, V], argmax tokens
        [T] int64)."""
        w = self.w
        tok = torch.as_tensor(tokens, dtype=torch.long).reshape(-1)
        T = tok.numel()
        pos = torch.arange(pos0, pos0 + T)
        n_q, n_kv, D = self.n_q, self.n_kv, self.D
        c, s = self.cos[pos][:, None, :], self.sin[pos][:, None, :]          # [T, 1, D/2]

        def rope(h):  # rope_ref per row at the row's own position (ref_ops.py:36-41)
            a, b = h[..., : D // 2].to(torch.float32), h[..., D // 2:].to(torch.float32)
            return torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(torch.float16)

        def proj(wm, x):  # gemv_ref of every row (ref_ops.py:10-12)
            return torch.mm(x.to(torch.float32), wm.to(torch.float32).t()).to(torch.float16)

        ctx = pos0 + T
        phys, slot = self.bt.to(torch.long)[pos // self.page], pos % self.page
        kvh = torch.arange(n_q) // (n_q // n_kv)
        causal = torch.arange(ctx)[None, :] > pos[:, None]                    # [T, ctx]: key after the row's position
        x = w["emb"][tok].clone()
        delta = None
        for li, lw in enumerate(w["layers"]):
            x, normed = R.add_rmsnorm_ref(x, delta, lw["ln1"], self.eps)
            qkv = proj(lw["qkv"], normed)
            q = rope(qkv[:, : n_q * D].reshape(T, n_q, D))
            k = rope(qkv[:, n_q * D:(n_q + n_kv) * D].reshape(T, n_kv, D))
            v = qkv[:, (n_q + n_kv) * D:].reshape(T, n_kv, D)
            kc, vc = self.kv[li, 0], self.kv[li, 1]
            kc[phys, :, slot, :] = k
            vc[phys, :, slot, :] = v
            kg, vg = R.gather_kv(kc, vc, self.bt, ctx, self.page)             # [ctx, n_kv, D]
            kf = kg.to(torch.float32)[:, kvh, :].permute(1, 0, 2)             # [n_q, ctx, D]
            vf = vg.to(torch.float32)[:, kvh, :].permute(1, 0, 2)
            sc = torch.bmm(q.to(torch.float32).permute(1, 0, 2), kf.transpose(1, 2).contiguous()) / math.sqrt(D)
            p = torch.softmax(sc.masked_fill(causal[None], float("-inf")), dim=-1)     # [n_q, T, ctx]
            attn = torch.bmm(p, vf).permute(1, 0, 2).to(torch.float16)         # [T, n_q, D]
            o = proj(lw["o"], attn.reshape(T, -1))
            x, normed = R.add_rmsnorm_ref(x, o, lw["ln2"], self.eps)
            act = R.swiglu_ref(proj(lw["gu"], normed))
            delta = proj(lw["down"], act)
        x, normed = R.add_rmsnorm_ref(x, delta, w["norm_f"], self.eps)
        logits = proj(w["lm_head"], normed)
        return logits, torch.argmax(logits.to(torch.float32), dim=-1)
