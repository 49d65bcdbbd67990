"""Batch-1 decode runtime for Llama-family models on one MI355X, built on the HIP decode kernels.

Mirrors the reference's ``runtime/model.py`` (DecodeConfig :32-50, Linear :56-72, Model :75-297): one decode step
(per layer)

    add_rmsnorm -> qkv GEMV -> RoPE + paged-KV append -> paged split-K attention (+ combine) -> o GEMV
    -> add_rmsnorm -> gate|up GEMV -> SwiGLU -> down GEMV

then the final add_rmsnorm -> LM head -> argmax into the device token slot -> pos += 1. State (token id, position)
lives in device tensors, so ``step()`` is captured once as a hipGraph (``torch.cuda.CUDAGraph`` on ROCm) and replayed
for every token. A prompt is either teacher-forced through the same graph, as in the reference, or processed in one
pass by ``prefill()`` (W4A16 MFMA GEMMs over all prompt rows, causal prefill attention), which leaves the same state.

Differences from the reference, all on the device side of the same composition:
  * head_dim 64 and 128 (TinyLlama and Llama-3-8B shapes);
  * the argmax and the position increment run as one kernel (dk_argmax_advance) instead of two torch ops;
  * weights are quantized on the GPU by the HIP RTN kernel;
  * there is no ``backend="ref"``: the CPU reference composition is test infrastructure (``oracle.decode_ref``);
  * the RoPE base is also found where transformers 5 keeps it (``rope_parameters``), and scaled RoPE types raise
    (``rope_theta_of``).

Knobs (DecodeConfig): weights "int4" | "fp16"; group; quant "rtn" | "clip" | "pre" (precomputed codes in qparams, e.g.
from runtime.gptq.calibrate); lm_head "auto" | "fp16" | "int4"; fused (False runs the
HF-style torch op sequences for norm and SwiGLU on the GPU, the reference's unfused comparison point); max_ctx, page,
part_size (0 -> attention policy table), attn_version, gemv_stage ((stage, R, warps, pf) forced everywhere, or None for
the tuning table), autotune_path, attn_policy_path, shuffle_pages, device; fused_attention, fused_gemv and swiglu
select the MI355X launch fusions (each one is checked against the unfused composition by the GPU tests).
"""
import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from . import ext
from .quant import QuantLinear

PKG = Path(__file__).resolve().parents[1]


@dataclass
class DecodeConfig:
    weights: str = "int4"
    group: int = 128
    quant: str = "rtn"             # "rtn" | "clip" (RTN with per-group range clipping, on the GPU) | "pre" (qparams)
    qparams: dict = field(default=None, repr=False)  # "layers.{i}.{qkv,o,gu,down}" / "lm_head" -> (q, scale, zero),
                                                     # e.g. runtime.gptq.calibrate
    lm_head: str = "auto"
    fused: bool = True
    backend: str = "hip"
    max_ctx: int = 2048
    page: int = 16
    part_size: int = 0
    attn_version: int = 0
    attn_impl: int = 0             # decode attention kernel: 0 = policy table, 1 = block kernel, 3 = lean MFMA
                                   # kernel (2, a removed MFMA kernel, runs the block kernel)
    gemv_stage: tuple = None
    autotune_path: str = str(PKG / "configs" / "autotune.json")
    attn_policy_path: str = str(PKG / "configs" / "attn_policy.json")
    shuffle_pages: bool = True
    device: str = "cuda"
    seed: int = 0            # block-table permutation seed
    fused_attention: bool = True   # rope_epilogue off: dk_attention_decode (RoPE + append in the split kernel) vs
                                   # rope_append + paged_attention
    argmax_split_min_v: int = 16384  # vocabularies at least this large pick the next token with the multi-workgroup
                                     # argmax (dk_argmax_advance_split); smaller ones with the one-workgroup kernel
    fused_gemv: bool = True        # residual + RMSNorm (and the embedding gather) computed inside the INT4 GEMV that
                                   # consumes it (dk_gemv_w4a16_rmsnorm) instead of a separate add_rmsnorm kernel
    f16_gemv: bool = True          # fp16-weight projections with K <= 4096 (the fp16 LM head) on the HIP fp16 GEMV
                                   # (dk_gemv_f16 / dk_gemv_f16_rmsnorm) instead of torch.mm
    rope_epilogue: bool = True     # with fused_gemv: RoPE + KV append in the qkv GEMV's epilogue
                                   # (dk_gemv_w4a16_qkv_rope over a rotation-pair copy of the qkv rows) and attention
                                   # without RoPE (dk_paged_attention) instead of dk_attention_decode; on MI355X
                                   # 1410 -> 1349 us per Llama-3-8B token at context 4096, unchanged on TinyLlama
    combine_in_o: bool = True      # with rope_epilogue: attention's split kernel alone (dk_paged_attention_split) and
                                   # its log-sum-exp combine merged by the o projection (dk_gemv_w4a16_attn) instead
                                   # of a combine launch, while every o workgroup's partials (splits x n_q x D fp32)
                                   # stay within Model.COMBINE_MAX_BYTES
    swiglu: str = "epilogue"       # where SwiGLU runs when fused_gemv is on: "epilogue" = inside the gate|up GEMV
                                   # (dk_gemv_w4a16_gate_up, gate/up rows stored interleaved); "kernel" = the separate
                                   # dk_swiglu launch


def rope_theta_of(config):
    """RoPE base of an HF-style config: its `rope_theta` attribute (transformers 4.x), else the "rope_theta" of its
    `rope_parameters` / `rope_scaling` dict (transformers 5.x keeps it only there), else 10000. The reference reads
    only the attribute (runtime/model.py:121) and so falls back to 10000 for a transformers-5 Llama-3 config (theta
    500000). Scaled RoPE variants (a rope_type other than "default", e.g. Llama-3.1's "llama3") are not implemented
    here and raise rather than rotate with the wrong frequencies."""
    theta = getattr(config, "rope_theta", None)
    params = getattr(config, "rope_parameters", None) or getattr(config, "rope_scaling", None)
    if isinstance(params, dict):
        rope_type = params.get("rope_type", params.get("type", "default"))
        if rope_type not in (None, "default"):
            raise NotImplementedError(f"rope_type {rope_type!r}: only the default (unscaled) RoPE is implemented")
        if theta is None:
            theta = params.get("rope_theta")
    return float(theta) if theta is not None else 10000.0


def default_gemv_config(N, K):
    """(stage, R, waves, pf) used when the tuning table has no entry for a shape (mirrors gemv_default_config in
    csrc/gemv_w4a16.hip): row tiles of 2 rows, one tile per workgroup (stage 4) while a workgroup can cover K
    (K <= 32768), split-K (stage 3) beyond."""
    if K <= 32768:
        return (4, 2, 0, 0)
    return (3, 2, 16, 1)


class Linear:
    """One projection in the format the config asks for (runtime/model.py:56-72).

    ``pairs_interleaved``: the rows of a [gate; up] stack are stored as gate_0, up_0, gate_1, up_1, ... (the layout
    dk_gemv_w4a16_gate_up reads); quantization is per row, so this is a pure row permutation of the stacked
    quantization. ``rows_reference_order`` undoes it for anything that needs the reference's row order."""

    def __init__(self, w, cfg: DecodeConfig, quant: bool, interleave_pairs: bool = False, key: str = None):
        self.N, self.K = w.shape
        self.quant = quant
        self.pairs_interleaved = interleave_pairs and quant
        dev = cfg.device
        if quant:
            if cfg.quant not in ("rtn", "clip", "pre"):
                raise ValueError(f"quant {cfg.quant!r}: 'rtn', 'clip' or 'pre'")
            pre = None
            if cfg.quant == "pre":
                pre = (cfg.qparams or {}).get(key)
                if pre is None:
                    raise ValueError(f"quant='pre': no precomputed codes for {key!r} in qparams")
            ql = QuantLinear(w.to(dev), cfg.group, clip=cfg.quant == "clip", qsz=pre)
            self.packed, self.sz = ql.packed, ql.sz
            self.nbytes = ql.nbytes()
            if self.pairs_interleaved:
                self.packed = interleave_halves(self.packed)
                self.sz = interleave_halves(self.sz)
        else:
            self.w = w.to(dev).half().contiguous()
            self.nbytes = self.w.numel() * 2

    def rows_reference_order(self, t):
        """A per-row tensor of this projection (dequantized weight, packed, sz) in the reference's [gate; up] order."""
        return deinterleave_halves(t) if self.pairs_interleaved else t


def rope_pair_rows(t, head_dim):
    """Rows of each head of a qkv stack [h*D + j] -> rotation pairs: row h*D + 2j = h*D + j, row h*D + 2j + 1 =
    h*D + j + D/2 (the layout dk_gemv_w4a16_qkv_rope reads)."""
    nh, half = t.size(0) // head_dim, head_dim // 2
    return t.view(nh, 2, half, *t.shape[1:]).transpose(1, 2).contiguous().view(t.shape)


def interleave_halves(t):
    """[a_0 .. a_{n-1}, b_0 .. b_{n-1}] rows -> [a_0, b_0, a_1, b_1, ...]."""
    n = t.size(0) // 2
    return t.view(2, n, *t.shape[1:]).transpose(0, 1).contiguous().view(t.shape)


def deinterleave_halves(t):
    n = t.size(0) // 2
    return t.view(n, 2, *t.shape[1:]).transpose(0, 1).contiguous().view(t.shape)


class Model:
    def __init__(self, hf_state, hf_config, cfg: DecodeConfig):
        self.cfg = cfg
        c = hf_config
        self.H, self.L = c.hidden_size, c.num_hidden_layers
        self.n_q, self.n_kv = c.num_attention_heads, c.num_key_value_heads
        self.D = self.H // self.n_q
        self.I, self.V = c.intermediate_size, c.vocab_size
        self.eps = c.rms_norm_eps
        if cfg.backend not in ("hip", "cuda"):
            raise ValueError(f"backend {cfg.backend!r}: this runtime runs the HIP kernels only; the CPU reference "
                             "composition is oracle.decode_ref (test infrastructure)")
        if self.D not in (64, 128):
            raise ValueError(f"head_dim {self.D} not supported (64 or 128)")
        if getattr(c, "head_dim", None) not in (None, self.D):
            raise ValueError(f"config head_dim {c.head_dim} != hidden_size / num_attention_heads = {self.D}")
        if getattr(c, "attention_bias", False) or getattr(c, "mlp_bias", False):
            raise NotImplementedError("projection biases (attention_bias / mlp_bias): the Llama composition this "
                                      "runtime implements has none")
        if getattr(c, "hidden_act", "silu") not in ("silu", "swish"):
            raise NotImplementedError(f"hidden_act {c.hidden_act!r}: the SwiGLU kernels implement silu only")
        self.rope_theta = rope_theta_of(c)   # raises for scaled RoPE types
        dev = cfg.device
        self.K = ext.load()
        quant = cfg.weights == "int4"
        if cfg.swiglu not in ("epilogue", "kernel"):
            raise ValueError(f"swiglu {cfg.swiglu!r}: 'epilogue' or 'kernel'")
        self.use_fused_gemv = (cfg.fused and cfg.fused_gemv and quant and self.H <= 32768 and self.I <= 32768)
        self.gate_up_epilogue = self.use_fused_gemv and cfg.swiglu == "epilogue"
        self.rope_epilogue = self.use_fused_gemv and cfg.rope_epilogue
        sd = hf_state
        g = lambda k: sd[k].half()
        self.emb = g("model.embed_tokens.weight").to(dev).contiguous()
        self.layers = []
        for i in range(self.L):
            p = f"model.layers.{i}."
            wqkv = torch.cat([g(p + "self_attn.q_proj.weight"), g(p + "self_attn.k_proj.weight"),
                              g(p + "self_attn.v_proj.weight")], 0)
            qkv = Linear(wqkv, cfg, quant, key=f"layers.{i}.qkv")
            del wqkv
            if self.rope_epilogue:  # decode-only copy; prefill reads the reference order
                qkv.rope_rows = (rope_pair_rows(qkv.packed, self.D), rope_pair_rows(qkv.sz, self.D))
            wgu = torch.cat([g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")], 0)
            gu = Linear(wgu, cfg, quant, interleave_pairs=self.gate_up_epilogue, key=f"layers.{i}.gu")
            del wgu
            self.layers.append({
                "ln1": g(p + "input_layernorm.weight").to(dev).contiguous(),
                "ln2": g(p + "post_attention_layernorm.weight").to(dev).contiguous(),
                "qkv": qkv, "o": Linear(g(p + "self_attn.o_proj.weight"), cfg, quant, key=f"layers.{i}.o"),
                "gu": gu, "down": Linear(g(p + "mlp.down_proj.weight"), cfg, quant, key=f"layers.{i}.down")})
        self.norm_f = g("model.norm.weight").to(dev).contiguous()
        lm = sd["lm_head.weight"] if "lm_head.weight" in sd else sd["model.embed_tokens.weight"]
        head_int4 = cfg.lm_head == "int4" or (cfg.lm_head == "auto" and quant)
        self.lm_head = Linear(lm.half(), cfg, head_int4, key="lm_head")

        self.gemv_table, self.gemv_norm_table, self.gemv_gate_up_table = {}, {}, {}
        self.gemv_f16_table, self.gemv_f16_norm_table = {}, {}
        self.gemv_us, self.gemv_norm_us = {}, {}
        self.step_cfg_override = {}
        if cfg.gemv_stage is None and Path(cfg.autotune_path).exists():
            tab = json.load(open(cfg.autotune_path))
            self.gemv_table = tab.get("best", {})
            self.gemv_norm_table = tab.get("best_norm", {})
            self.gemv_us, self.gemv_norm_us = tab.get("us", {}), tab.get("us_norm", {})
            self.gemv_gate_up_table = tab.get("best_gate_up", {})
            self.gemv_f16_table = tab.get("best_f16", {})
            self.gemv_f16_norm_table = tab.get("best_f16_norm", {})
            # configurations chosen by the decode step time (runtime.autotune.tune_step), ahead of the isolated tables
            self.step_cfg_override = {k: tuple(v) for k, v in tab.get("best_step", {}).items()}

        # paged KV cache [L, 2, pages, n_kv, P, D]; one block table shared by all layers (one sequence)
        self.n_pages = (cfg.max_ctx + cfg.page - 1) // cfg.page + 1
        self.kv = torch.zeros(self.L, 2, self.n_pages, self.n_kv, cfg.page, self.D, dtype=torch.half, device=dev)
        gen = torch.Generator().manual_seed(cfg.seed)
        perm = torch.randperm(self.n_pages, generator=gen) if cfg.shuffle_pages else torch.arange(self.n_pages)
        self.bt = perm.int().to(dev)
        self.cos, self.sin = (t.to(dev) for t in rope_tables(cfg.max_ctx + 1, self.D, self.rope_theta))

        self.attn_version = cfg.attn_version or self._policy().get("version", 3)
        self.set_attention_partition(cfg.max_ctx)

        h16 = dict(dtype=torch.half, device=dev)
        self.tok = torch.zeros(1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.x = torch.empty(self.H, **h16)
        self.x_alt = torch.empty(self.H, **h16)    # second residual buffer of the fused-prologue step
        self.normed = torch.empty(self.H, **h16)
        self.qkv = torch.empty((self.n_q + 2 * self.n_kv) * self.D, **h16)
        self.attn = torch.empty(self.n_q, self.D, **h16)
        self.o = torch.empty(self.H, **h16)
        self.gu = torch.empty(2 * self.I, **h16)
        self.act = torch.empty(self.I, **h16)
        self.down = torch.empty(self.H, **h16)
        self.logits = torch.empty(self.V, **h16)
        # meeting point of the multi-workgroup argmax: zero here, left zero by every launch
        self.argmax_work = torch.zeros(2, dtype=torch.int64, device=self.cfg.device)
        self.graph = None
        self.host_pos = 0

    # ------------------------------------------------------------------ helpers
    def set_attention_partition(self, ctx_cap, part_size=None, impl=None):
        """Choose the attention kernel and split size for contexts up to ctx_cap (explicit arguments, then the
        config, then the policy entry tuned for the largest context <= ctx_cap) and allocate the split partials for
        a grid of ceil(ctx_cap / part_size) splits; splits past the live context exit at once. The effective cap is
        rounded up to whole splits and guarded by run_step (the behaviour of runtime/model.py:140-151)."""
        ent = self._policy_entry(ctx_cap)
        ps = part_size or self.cfg.part_size or ent.get("part_size", 64)
        impl = impl or self.cfg.attn_impl or ent.get("impl", 1)
        if impl == 2:
            impl = 1                                # tables written before the MFMA kernel's removal
        lean_max = 256 if self.D == 128 else 512
        if impl == 3 and (self.cfg.page < 16 or ps % 16 or ps > lean_max):
            impl = 1                                # the lean kernel takes whole 16-token tiles of one page
        splits = -(-ctx_cap // ps)
        self.attn_impl, self.part_size, self.max_splits, self.ctx_cap = impl, ps, max(1, splits), max(1, splits) * ps
        # the o projection merges the split partials itself (one thread per 8 values of x, at most 8 waves) while
        # the partials one of its workgroups reads (every split of all of x) stay small
        self.attn_in_o = (self.cfg.combine_in_o and self.rope_epilogue and self.layers[0]["o"].quant
                          and self.max_splits <= self.COMBINE_MAX_SPLITS and self.n_q * self.D <= 4096
                          and self.max_splits * self.n_q * self.D * 4 <= self.COMBINE_MAX_BYTES)
        dev = self.cfg.device
        self.o_part, self.m_part, self.l_part = (
            torch.empty(*shape, dtype=torch.float32, device=dev)
            for shape in ((self.n_q, self.max_splits, self.D), (self.n_q, self.max_splits), (self.n_q, self.max_splits)))
        self.graph = None

    def prepare(self, ctx_cap, use_graph=True, part_size=None, impl=None):
        """Configure attention for contexts <= ctx_cap and (re)capture the decode graph (runtime/model.py:153-158)."""
        if ctx_cap > self.cfg.max_ctx:
            raise ValueError(f"prepare: context cap {ctx_cap} exceeds the cache's max_ctx {self.cfg.max_ctx}")
        self.set_attention_partition(ctx_cap, part_size, impl)
        if use_graph:
            self.capture()

    def _policy(self):
        p = Path(self.cfg.attn_policy_path)
        return json.load(open(p)) if p.exists() else {}

    def _policy_entry(self, ctx_cap):
        return self._policy_entry_of(self._policy(), self.D, ctx_cap)

    @staticmethod
    def _policy_entry_of(pol, head_dim, ctx_cap):
        """Entry tuned at the largest context <= ctx_cap (runtime/model.py:164-172), from the head-dim-specific table
        ("policy_d128") when there is one: {"part_size", "impl"}."""
        ents = [e for e in pol.get(f"policy_d{head_dim}", pol.get("policy", [])) if e["max_ctx"] < (1 << 30)]
        if not ents:
            return {"part_size": 64, "impl": 1}
        below = [e for e in ents if e["max_ctx"] <= ctx_cap]
        return below[-1] if below else ents[0]

    def step_key(self, kind, lin):
        """Key of the in-step tuning table: "kind:NxK_G" (INT4) or "kind:NxK" (fp16)."""
        return f"{kind}:{lin.N}x{lin.K}" + (f"_G{self.cfg.group}" if lin.quant else "")

    def gemv_cfg(self, lin):
        if self.cfg.gemv_stage is not None:
            return self.cfg.gemv_stage
        e = self.step_cfg_override.get(self.step_key("plain", lin))
        if e is not None:
            return tuple(e)
        e = self.gemv_table.get(f"{lin.N}x{lin.K}_G{self.cfg.group}")
        if e is None:
            return default_gemv_config(lin.N, lin.K)
        return tuple(e) if len(e) == 4 else (2, *e)      # [R, warps, pf] is the reference's stage-2 schema

    def gemv_norm_cfg(self, lin):
        """Configuration of the fused-norm GEMV: its own tuned entry (every workgroup recomputes the norm, so larger
        row tiles pay off), else 4-row tiles."""
        e = self.step_cfg_override.get(self.step_key("norm", lin))
        if e is None:
            e = self.gemv_norm_table.get(f"{lin.N}x{lin.K}_G{self.cfg.group}")
        return tuple(e) if e is not None else (4, 4, 0, 1)

    # in-graph time of the separate add_rmsnorm launch at hidden 2048-4096 on MI355X (decode-step kernel trace)
    ADD_RMSNORM_US = 2.5
    COMBINE_MAX_SPLITS = 16            # dk_gemv_w4a16_attn merges at most this many splits
    # partial bytes per o workgroup up to which the merge pays on MI355X: TinyLlama ctx 512, part 128 (5 splits, 40 KB)
    # 530 -> 504 us per step; Llama-3-8B ctx 1024, part 128 (9 splits, 144 KB) 1266 -> 1528
    COMBINE_MAX_BYTES = 64 << 10

    def gemv_attn_cfg(self, lin):
        """Configuration of the o projection with the attention combine in its prologue: its in-step entry ("attn:"
        key), else 1-row tiles, 2 per row group, and the fewest waves that give every 8 values of x a thread."""
        tw = -(-lin.K // 2048)
        need = -(-max(-(-lin.K // 512), tw) // tw) * tw
        e = self.step_cfg_override.get(self.step_key("attn", lin))
        s, r, wv, pf = tuple(e) if e is not None else (4, 1, need, 1)
        return 4, r, max(wv, need), pf

    def norm_fusion_pays(self, lin):
        """Whether the residual + RMSNorm should run inside this INT4 GEMV: the tuned fused time against the tuned
        plain GEMV plus a separate add_rmsnorm. Every workgroup of the fused kernel recomputes the norm over K, which
        loses on the widest shapes (e.g. the 128256 x 4096 INT4 head, where split-K wins)."""
        key = f"{lin.N}x{lin.K}_G{self.cfg.group}"
        fused, plain = self.gemv_norm_us.get(key), self.gemv_us.get(key)
        return fused is None or plain is None or fused <= plain + self.ADD_RMSNORM_US

    def linear_norm(self, lin: Linear, x_in, delta, w, x_out, y, row=None):
        """y = W . rmsnorm(x_in + delta) with x_out <- x_in + delta, one launch (dk_gemv_w4a16_rmsnorm)."""
        s, r, wv, pf = self.gemv_norm_cfg(lin)
        self.K.gemv_w4a16_rmsnorm(s, r, wv, pf, lin.packed, lin.sz, x_in, row, delta, w, self.eps, x_out, y,
                                  self.cfg.group)

    def gemv_gate_up_cfg(self, lin):
        """Configuration of the gate|up GEMV with the SwiGLU epilogue: its tuned entry, else the fused-norm one; the
        row tile R * 2^pf must hold a gate/up pair."""
        key = f"{lin.N}x{lin.K}_G{self.cfg.group}"
        e = (self.step_cfg_override.get(self.step_key("gate_up", lin)) or self.gemv_gate_up_table.get(key)
             or self.gemv_norm_table.get(key) or (4, 4, 0, 1))
        s, r, wv, pf = e
        if (r << pf) < 2:
            r = 2
        return s, r, wv, pf

    def linear_gate_up(self, lin: Linear, x_in, delta, w, x_out, act):
        """act = swiglu(W_gu . rmsnorm(x_in + delta)) with x_out <- x_in + delta, one launch (dk_gemv_w4a16_gate_up
        over the interleaved gate/up rows)."""
        s, r, wv, pf = self.gemv_gate_up_cfg(lin)
        self.K.gemv_w4a16_gate_up(s, r, wv, pf, lin.packed, lin.sz, x_in, None, delta, w, self.eps, x_out, act,
                                  self.cfg.group)

    def use_f16_gemv(self, lin):
        return self.cfg.fused and self.cfg.f16_gemv and not lin.quant and lin.K <= 4096 and lin.K % 8 == 0

    def gemv_f16_cfg(self, lin, norm=False):
        """(R, waves, pf) of the fp16 GEMV (norm: the variant behind the final RMSNorm): tuned entry, else 2-row tiles
        (1 for K > 2048), 1 wave per workgroup, 4 tiles per wave."""
        e = self.step_cfg_override.get(self.step_key("f16_norm", lin)) if norm else None
        if e is None:
            e = (self.gemv_f16_norm_table if norm else self.gemv_f16_table).get(f"{lin.N}x{lin.K}")
        return tuple(e) if e is not None else ((2 if lin.K <= 2048 else 1), 1, 2)

    def linear(self, lin: Linear, x, y):
        if lin.quant:
            s, r, w, pf = self.gemv_cfg(lin)
            self.K.gemv_w4a16(s, r, w, pf, lin.packed, lin.sz, x, y, self.cfg.group)
        elif self.use_f16_gemv(lin):
            self.K.gemv_f16(*self.gemv_f16_cfg(lin), lin.w, x, y)
        else:
            torch.mm(x.view(1, -1), lin.w.t(), out=y.view(1, -1))  # rocBLAS / hipBLASLt, the reference's cuBLAS call

    def add_norm(self, delta, w):
        if self.cfg.fused:
            self.K.add_rmsnorm(self.x, delta, w, self.normed, self.eps)
        else:  # HF op sequence on the GPU (the reference's unfused comparison point)
            if delta is not None:
                self.x.add_(delta)
            xf = self.x.float()
            self.normed.copy_(w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).half())

    def swiglu(self):
        if self.cfg.fused:
            self.K.swiglu(self.gu, self.act)
        else:
            self.act.copy_(torch.nn.functional.silu(self.gu[: self.I].float()).half() * self.gu[self.I:])

    def pick_next(self):
        """tok <- argmax(logits), pos += 1 (runtime/model.py:232-233) in one launch."""
        if self.V >= self.cfg.argmax_split_min_v:
            self.K.argmax_advance_split(self.logits, self.tok, self.pos, self.argmax_work)
        else:
            self.K.argmax_advance(self.logits, self.tok, self.pos)

    def qkv_rope_cfg(self, lin):
        """Row tile of the qkv GEMV with the RoPE + append epilogue: its in-step entry ("rope:" key, written by
        runtime.autotune.tune_step), else the fused-norm one; a tile (R * 2^pf rows) must hold a rotation pair."""
        e = self.step_cfg_override.get(self.step_key("rope", lin))
        _, r, wv, pf = tuple(e) if e is not None else self.gemv_norm_cfg(lin)
        if (r << pf) < 2:
            r = 2
        return 4, r, wv, pf

    def qkv_proj(self, lin: Linear, li, x_in, delta, w, x_out, row=None):
        """qkv = W_qkv . x (w None: x is the normed input) or W_qkv . rmsnorm(x_in + delta); with the RoPE epilogue
        the same launch also rotates q and appends k, v to layer li's cache."""
        if not self.rope_epilogue:
            if w is None:
                self.linear(lin, x_in, self.qkv)
            else:
                self.linear_norm(lin, x_in, delta, w, x_out, self.qkv, row=row)
            return
        _, r, wv, pf = self.qkv_rope_cfg(lin)
        packed, sz = lin.rope_rows
        self.K.gemv_w4a16_qkv_rope(4, r, wv, pf, packed, sz, x_in, row, delta, w, self.eps, x_out, self.qkv, self.cos,
                                   self.sin, self.pos, self.bt, self.kv[li, 0], self.kv[li, 1], self.n_q, self.n_kv,
                                   self.cfg.group)

    def attention(self, li):
        kc, vc = self.kv[li, 0], self.kv[li, 1]
        if self.rope_epilogue:  # q rotated and k, v appended by the qkv GEMV
            version = 5 if self.attn_impl == 3 else 4     # the policy's kernel, explicitly
            if self.attn_in_o:  # the o projection merges the partials
                self.K.paged_attention_split(self.qkv[: self.n_q * self.D], kc, vc, self.bt, self.pos,
                                             self.part_size, self.o_part, self.m_part, self.l_part, self.attn, version)
                return
            self.K.paged_attention(self.qkv[: self.n_q * self.D], kc, vc, self.bt, self.pos, self.part_size,
                                   self.o_part, self.m_part, self.l_part, self.attn, version)
            return
        if self.cfg.fused_attention:
            self.K.attention_decode(self.qkv, self.cos, self.sin, self.pos, self.bt, kc, vc, self.n_q, self.n_kv,
                                    self.part_size, self.o_part, self.m_part, self.l_part, self.attn, self.attn_impl)
            return
        self.K.rope_append(self.qkv, self.cos, self.sin, self.pos, self.bt, kc, vc, self.n_q, self.n_kv)
        self.K.paged_attention(self.qkv[: self.n_q * self.D], kc, vc, self.bt, self.pos, self.part_size,
                               self.o_part, self.m_part, self.l_part, self.attn, self.attn_version)

    # ------------------------------------------------------------------ decode step
    def step(self):
        """One token: reads tok/pos, writes logits, tok <- argmax, pos += 1 (runtime/model.py:216-233)."""
        if self.use_fused_gemv:
            self.step_fused()
            return
        torch.index_select(self.emb, 0, self.tok, out=self.x.view(1, -1))
        delta = None
        for li, lw in enumerate(self.layers):
            self.add_norm(delta, lw["ln1"])
            self.linear(lw["qkv"], self.normed, self.qkv)
            self.attention(li)
            self.linear(lw["o"], self.attn.view(-1), self.o)
            self.add_norm(self.o, lw["ln2"])
            self.linear(lw["gu"], self.normed, self.gu)
            self.swiglu()
            self.linear(lw["down"], self.act, self.down)
            delta = self.down
        self.add_norm(delta, self.norm_f)
        self.linear(self.lm_head, self.normed, self.logits)
        self.pick_next()

    def step_fused(self):
        """The same composition with every residual + RMSNorm inside the GEMV that consumes it (the layer-0 one also
        gathers the embedding row of the device token) and, by default, SwiGLU in the gate|up GEMV's epilogue: per
        layer qkv, attention (split + combine), o, gate|up, down = 6 launches, 5 when the o projection merges the
        attention's split partials itself (attn_in_o). The residual stream alternates between
        two buffers because a fused GEMV's workgroups all read x_in while workgroup 0 writes x_in + delta."""
        cur, nxt = self.x, self.x_alt
        delta = None
        for li, lw in enumerate(self.layers):
            if li == 0:
                self.qkv_proj(lw["qkv"], li, self.emb, None, lw["ln1"], cur, row=self.tok)
            elif self.norm_fusion_pays(lw["qkv"]):
                self.qkv_proj(lw["qkv"], li, cur, delta, lw["ln1"], nxt)
                cur, nxt = nxt, cur
            else:
                self.K.add_rmsnorm(cur, delta, lw["ln1"], self.normed, self.eps)
                self.qkv_proj(lw["qkv"], li, self.normed, None, None, None)
            self.attention(li)
            if self.attn_in_o:
                s, r, wv, pf = self.gemv_attn_cfg(lw["o"])
                self.K.gemv_w4a16_attn(s, r, wv, pf, lw["o"].packed, lw["o"].sz, self.o_part, self.m_part,
                                       self.l_part, self.attn, self.pos, self.bt, self.cfg.page, self.part_size, 0,
                                       self.o, self.cfg.group)
            else:
                self.linear(lw["o"], self.attn.view(-1), self.o)
            if self.gate_up_epilogue:
                self.linear_gate_up(lw["gu"], cur, self.o, lw["ln2"], nxt, self.act)
                cur, nxt = nxt, cur
                self.linear(lw["down"], self.act, self.down)
            else:
                self.linear_norm(lw["gu"], cur, self.o, lw["ln2"], nxt, self.gu)
                cur, nxt = nxt, cur
                self.K.swiglu(self.gu, self.act)
                self.linear(lw["down"], self.act, self.down)
            delta = self.down
        if self.lm_head.quant and self.norm_fusion_pays(self.lm_head):
            self.linear_norm(self.lm_head, cur, delta, self.norm_f, None, self.logits)
        elif self.use_f16_gemv(self.lm_head):
            self.K.gemv_f16_rmsnorm(*self.gemv_f16_cfg(self.lm_head, norm=True), self.lm_head.w, cur, delta,
                                    self.norm_f, self.eps, None, self.logits)
        else:
            self.K.add_rmsnorm(cur, delta, self.norm_f, self.normed, self.eps)
            self.linear(self.lm_head, self.normed, self.logits)
        self.pick_next()

    def _keep_state(self):
        """Context manager: the device token and position as they are now, put back on exit."""
        model = self

        class _Keep:
            def __enter__(self):
                self.saved = torch.cat([model.tok, model.pos.to(torch.long)])
                return self

            def __exit__(self, *exc):
                model.tok.copy_(self.saved[:1])
                model.pos.copy_(self.saved[1:].to(torch.int32))
                return False

        return _Keep()

    def capture(self):
        """Record step() into a hipGraph (torch.cuda.CUDAGraph), the role of runtime/model.py:235-251: two warm-up
        steps run on a side stream at position 0 (the split buffers are sized for the prepared cap, which a stale
        position could exceed; the K/V the warm-up writes sit at positions every real step overwrites before reading),
        then one step is recorded. Token and position are left as they were."""
        with self._keep_state():
            self.pos.zero_()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self.step()
                self.step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.step()
            self.graph = graph
        torch.cuda.synchronize()

    def _claim_positions(self, n):
        """Account for n more steps on the host and refuse them if attention was not prepared that far (tokens past
        the cap would silently not be attended)."""
        end = self.host_pos + n
        if end > self.ctx_cap:
            raise RuntimeError(f"context {end} exceeds the prepared attention cap {self.ctx_cap}; call prepare()")
        self.host_pos = end

    def run_step(self, use_graph=True):
        """One token through the captured graph (or eagerly without one)."""
        self._claim_positions(1)
        (self.graph.replay if use_graph and self.graph is not None else self.step)()

    # ------------------------------------------------------------------ high level
    def reset(self, pos=0):
        """Start a sequence at position pos (device and host mirror); the cache below pos is kept."""
        self.host_pos = int(pos)
        self.pos.fill_(self.host_pos)

    def teacher_force(self, tokens, use_graph=True, collect_logits=False):
        """Step through the given token ids (each fed as the step's input token) from the current position; returns
        the logits of every step (fp16 [len, V]) when collect_logits is set."""
        ids = torch.as_tensor(tokens, dtype=torch.long).reshape(-1).to(self.tok.device)
        if ids.numel() and not bool(((ids >= 0) & (ids < self.V)).all()):
            raise ValueError(f"teacher_force: token ids must lie in [0, {self.V})")  # they index embedding rows
        rows = []
        for t in range(ids.numel()):
            self.tok.copy_(ids[t:t + 1])
            self.run_step(use_graph)
            if collect_logits:
                rows.append(self.logits.clone())
        if not collect_logits:
            return None
        return torch.stack(rows) if rows else torch.empty(0, self.V, dtype=torch.half, device=self.tok.device)

    def _prefill_buffers(self, M):
        if getattr(self, "_pf_rows", 0) < M:
            h16 = dict(dtype=torch.half, device=self.cfg.device)
            self._pf_rows = M
            self._pf = {"x": torch.empty(M, self.H, **h16), "xn": torch.empty(M, self.H, **h16),
                        "qkv": torch.empty(M, (self.n_q + 2 * self.n_kv) * self.D, **h16),
                        "attn": torch.empty(M, self.n_q * self.D, **h16), "o": torch.empty(M, self.H, **h16),
                        "act": torch.empty(M, self.I, **h16), "down": torch.empty(M, self.H, **h16),
                        "tok": torch.empty(M, dtype=torch.long, device=self.cfg.device)}
        return {k: v[:M] for k, v in self._pf.items()}

    def gemm(self, lin: Linear, x, y, epilogue=0):
        """Y [M, N] = X [M, K] . W^T for M prompt rows: the W4A16 GEMM for packed weights, rocBLAS / hipBLASLt for
        fp16 ones (the reference's cuBLAS call for an fp16 projection)."""
        if lin.quant:
            if epilogue == 1:
                packed, sz = self._gate_up_pairs(lin)
                self.K.gemm_w4a16(packed, sz, x, y, self.cfg.group, epilogue=1)
            else:
                self.K.gemm_w4a16(lin.packed, lin.sz, x, y, self.cfg.group,
                                  workspace=self._gemm_workspace(x.size(0), lin.N, lin.K))
        else:
            torch.mm(x, lin.w.t(), out=y)

    def _gemm_workspace(self, M, N, K):
        """The split-K workspace of the projections that do not fill the CUs unsplit (None where a shape does not
        split); one buffer for the model, grown to the largest need seen."""
        need = self.K.gemm_workspace_bytes(M, N, K, self.cfg.group)
        if need == 0:
            return None
        if getattr(self, "_gws", None) is None or self._gws.numel() < need:
            self._gws = torch.empty(need, dtype=torch.uint8, device=self.cfg.device)
        return self._gws

    # prefill projections whose output only feeds the next residual + RMSNorm (o, down): where the GEMM splits K, its
    # fp32 partials go straight to the norm, which sums them as the GEMM's reduce launch would (bit for bit the same
    # x and normed rows, one launch fewer)
    fold_split_reduce = True

    def _proj_delta(self, lin, x_in, y):
        """Y = X . W^T of such a projection: the split partials [S, M, N] (a view of the workspace, valid until the
        next GEMM that splits) where the shape splits, else y itself."""
        if lin.quant and self.fold_split_reduce:
            ws = self._gemm_workspace(x_in.size(0), lin.N, lin.K)
            if ws is not None:
                return self.K.gemm_w4a16_parts(lin.packed, lin.sz, x_in, self.cfg.group, ws)
        self.gemm(lin, x_in, y)
        return y

    def _add_norm_rows(self, x, delta, w, xn):
        """x += delta (fp16 rows, or split partials [S, M, H]); xn = RMSNorm(x) * w, in place over the prompt rows."""
        if delta.dtype == torch.float32:
            self.K.rmsnorm_rows_parts(x, delta, w, x, xn, self.eps)
        else:
            self.K.rmsnorm_rows(x, None, delta, w, x, xn, self.eps)

    def _gate_up_pairs(self, lin):
        """Interleaved (gate_i, up_i) rows for the GEMM's SwiGLU epilogue: the Linear's own storage when the decode
        step already uses that layout, else a permuted copy made once."""
        if lin.pairs_interleaved:
            return lin.packed, lin.sz
        if not hasattr(lin, "_il"):
            lin._il = (interleave_halves(lin.packed), interleave_halves(lin.sz))
        return lin._il

    def prefill(self, tokens):
        """Process a prompt in one pass: every projection of the M tokens is one W4A16 GEMM, rope/append and the
        residual + RMSNorm run over all rows, attention is causal over the paged cache (row m at position pos + m).
        Leaves the state teacher_force(tokens) leaves -- the cache rows of positions pos .. pos + M - 1 written,
        logits of the last token, tok = their argmax, pos += M -- up to the summation order of the GEMM (the
        reference teacher-forces prompts through its decode step, runtime/model.py:278-286; this is the batched form
        of the same composition, runtime/model.py:216-233 per row)."""
        toks = torch.as_tensor(tokens).long().flatten()
        M = toks.numel()
        if M == 0:
            return
        if int(toks.min()) < 0 or int(toks.max()) >= self.V:
            raise ValueError(f"prefill: token ids must lie in [0, {self.V})")
        start = self.host_pos
        if start + M > self.cfg.max_ctx:
            raise RuntimeError(f"prefill: context {start + M} exceeds max_ctx {self.cfg.max_ctx}")
        B = self._prefill_buffers(M)
        B["tok"].copy_(toks)
        x, xn, delta = B["x"], B["xn"], None
        eps = self.eps
        for li, lw in enumerate(self.layers):
            if li == 0:
                self.K.rmsnorm_rows(self.emb, B["tok"], None, lw["ln1"], x, xn, eps)
            else:
                self._add_norm_rows(x, delta, lw["ln1"], xn)
            self.gemm(lw["qkv"], xn, B["qkv"])
            kc, vc = self.kv[li, 0], self.kv[li, 1]
            self.K.rope_append_rows(B["qkv"], self.cos, self.sin, self.pos, self.bt, kc, vc, self.n_q, self.n_kv)
            self.K.attention_prefill(B["qkv"], self.pos, self.bt, kc, vc, self.n_q, self.n_kv, start + M, B["attn"])
            self._add_norm_rows(x, self._proj_delta(lw["o"], B["attn"], B["o"]), lw["ln2"], xn)
            if lw["gu"].quant:
                self.gemm(lw["gu"], xn, B["act"], epilogue=1)
            else:
                gu = torch.mm(xn, lw["gu"].w.t())
                B["act"].copy_(torch.nn.functional.silu(gu[:, : self.I].float()).half() * gu[:, self.I:])
            delta = self._proj_delta(lw["down"], B["act"], B["down"])
        last = slice(M - 1, M)
        self._add_norm_rows(x[last], delta[:, last] if delta.dtype == torch.float32 else delta[last], self.norm_f,
                            xn[last])
        self.linear(self.lm_head, xn[M - 1], self.logits)
        if M > 1:
            self.pos.add_(M - 1)
        self.pick_next()
        self.host_pos = start + M

    def generate(self, prompt, n_new, use_graph=True, prefill=False):
        """Greedy decoding from position 0 (runtime/model.py:278-286): the prompt teacher-forced (or prefilled in one
        pass), then n_new tokens. The tokens are gathered on the device and read back once at the end."""
        self.reset(0)
        (self.prefill if prefill else lambda p: self.teacher_force(p, use_graph))(prompt)
        picked = torch.empty(max(n_new, 1), dtype=torch.long, device=self.tok.device)
        picked[:1].copy_(self.tok)
        for i in range(1, n_new):
            self.run_step(use_graph)
            picked[i:i + 1].copy_(self.tok)
        return picked[:n_new].tolist()

    # ------------------------------------------------------------------ byte accounting (roofline)
    def _projections(self):
        for lw in self.layers:
            yield from (lw[k] for k in ("qkv", "o", "gu", "down"))

    def weight_bytes(self):
        """Bytes of weights one token reads, from the built tensors: every projection of the body with the two norm
        vectors per layer, the LM head, and one embedding row (the byte model of runtime/model.py:289-297)."""
        norms = sum(lw[k].numel() * lw[k].element_size() for lw in self.layers for k in ("ln1", "ln2"))
        return {"body": sum(p.nbytes for p in self._projections()) + norms, "lm_head": self.lm_head.nbytes,
                "embedding_row": self.emb[0].numel() * self.emb.element_size()}

    def kv_bytes_per_token(self, ctx):
        """K and V bytes of all layers that one token moves: ctx cached rows read, one new row written."""
        row = self.kv[0, 0, 0, :, 0].numel() * self.kv.element_size()    # one token's K (or V) of one layer
        return 2 * row * self.L * (ctx + 1)

    def activation_bytes(self):
        """fp16 activation vectors read/written per token (bench/analyze.py:40 of the reference)."""
        return 2 * (self.L * (self.H * 6 + self.I * 3 + (self.n_q + 2 * self.n_kv) * self.D) + self.V)

    def bytes_per_token(self, ctx):
        w = self.weight_bytes()
        return w["body"] + w["lm_head"] + w["embedding_row"] + self.kv_bytes_per_token(ctx) + self.activation_bytes()


def byte_model(shape, ctx, group=128, head="fp16", weights="int4"):
    """Algorithmic bytes one decode token moves at context ctx, from the shape alone (the byte model of
    runtime/model.py:289-297 and bench/analyze.py:35-40 of the reference): the projections (INT4: packed N K / 2 plus
    (scale, zero) 4 N K / G each; fp16: 2 N K) and the two fp16 norm weights of every layer, the LM head (fp16 or
    INT4), one embedding row, the KV cache read for ctx tokens and written for one, and the fp16 activation vectors.
    Model.bytes_per_token gives the same total from the built tensors. Returns the parts and "total"."""
    H, L, I, V = shape.hidden_size, shape.num_hidden_layers, shape.intermediate_size, shape.vocab_size
    n_q, n_kv = shape.num_attention_heads, shape.num_key_value_heads
    D = H // n_q

    def lin(N, K, fmt):
        return N * K // 2 + 4 * N * (K // group) if fmt == "int4" else 2 * N * K

    body = L * (lin((n_q + 2 * n_kv) * D, H, weights) + lin(H, n_q * D, weights) + lin(2 * I, H, weights)
                + lin(H, I, weights) + 2 * 2 * H)
    row = n_kv * D * 2
    parts = {"body": body, "lm_head": lin(V, H, head), "embedding_row": 2 * H,
             "kv": L * (2 * row * ctx + 2 * row),
             "activations": 2 * (L * (H * 6 + I * 3 + (n_q + 2 * n_kv) * D) + V)}
    parts["total"] = sum(parts.values())
    return parts


def rope_tables(max_pos, head_dim, theta=10000.0, device="cpu"):
    """fp32 (cos, sin) [max_pos, head_dim/2] of angles p * theta^(-2i/head_dim) computed in float64
    (reference/ref_ops.py:30-33)."""
    i2 = torch.arange(0, head_dim, 2, dtype=torch.float64, device=device)
    inv_freq = 1.0 / torch.pow(torch.tensor(float(theta), dtype=torch.float64, device=device), i2 / head_dim)
    ang = torch.arange(max_pos, dtype=torch.float64, device=device)[:, None] * inv_freq[None, :]
    return ang.cos().float().contiguous(), ang.sin().float().contiguous()
