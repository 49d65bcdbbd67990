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
"""
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
