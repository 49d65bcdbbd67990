"""Full-depth decode parity: the graph-captured HIP decode step of the BASELINE models at their real size against the
CPU oracle decoder (oracle/decode_ref.py, the reference's backend="ref" composition, runtime/model.py:216-233).

  * config 4: TinyLlama-1.1B architecture (22 layers, hidden 2048, 32 q / 4 kv heads, head_dim 64, SwiGLU 5632,
    vocab 32000), INT4 G128 body, fp16 LM head, contexts 512 and 2048, 16 greedy steps each;
  * config 5: Llama-3-8B architecture (32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 14336,
    vocab 128256, rope theta 5e5), INT4 G128 body and LM head, context 4096, 6 greedy steps.

Both decoders start from the same state: positions 0 .. ctx-1 of every layer's K and V cache hold the same seeded
N(0, 1) values (filling them by teacher forcing would cost the CPU minutes per context), then each step feeds the same
token to both, the GPU's own greedy choice from the step before. The oracle's weights are the model's INT4 codes
dequantized by the oracle (quant_ref.dequantize_packed, pinned bit-exact to the numpy restatement on the CPU; here it
runs on the GPU's tensors so that the 8B model's 7.5 G weights dequantize in seconds, and a sampled block of rows is
checked against the numpy path) and held as float32 copies of their fp16 values on the CPU.

Bars (the reference's, tests/test_kernels.py and tests/test_runtime_local.py:21-28):
  * logits of every step within 2e-2 normwise (the whole-step bar of the golden decode test);
  * greedy agreement: the GPU's argmax equals the oracle's, except where the oracle's top1 - top2 margin is within
    4x that step's largest logit difference (a near-tie the observed error can flip; the margin is reported);
  * the K and V rows the step appends at positions ctx .. ctx+steps-1 within 2e-2 normwise of the oracle's.
"""
import numpy as np
import pytest
import torch

from helpers import err
from oracle import quant_ref as Q
from oracle.decode_ref import RefDecoder

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def oracle_weights(m):
    """{emb, norm_f, lm_head, layers[...]} for RefDecoder: float32 CPU copies of the fp16 weights the reference's ref
    backend computes with (INT4 projections dequantized from the model's packed codes, in the reference's row order)."""
    g = m.cfg.group

    def deq(lin):
        if not lin.quant:
            return lin.w.cpu().float()
        packed, sz = lin.rows_reference_order(lin.packed), lin.rows_reference_order(lin.sz)
        w = Q.dequantize_packed(packed, sz, g)
        rows = slice(0, min(64, lin.N))                 # spot check of the device run against the numpy path
        want = Q.dequantize(Q.unpack(packed[rows].cpu().numpy()), *Q.unpack_scale_zero(sz[rows].cpu().numpy()), g)
        assert np.array_equal(w[rows].cpu().numpy().view(np.uint16), want.view(np.uint16))
        return w.cpu().float()

    return {"emb": m.emb.cpu(), "norm_f": m.norm_f.cpu(), "lm_head": deq(m.lm_head),
            "layers": [{"ln1": l["ln1"].cpu(), "ln2": l["ln2"].cpu(), "qkv": deq(l["qkv"]), "o": deq(l["o"]),
                        "gu": deq(l["gu"]), "down": deq(l["down"])} for l in m.layers]}


def fill_cache(m, ref, seed):
    """The same seeded N(0, 1) fp16 values in every page of both caches (the GPU cache and the oracle's share the
    block table, so token t of layer l is the same vector in both)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    for li in range(m.L):
        m.kv[li].copy_(torch.randn(m.kv[li].shape, generator=g, device=DEV, dtype=torch.float32).half())
    ref.kv.copy_(m.kv.cpu())


def appended_rows(kv, bt, page, lo, hi):
    """K and V rows of positions lo .. hi-1 of every layer: [L, 2, hi - lo, n_kv, D]."""
    t = torch.arange(lo, hi)
    return kv[:, :, bt[t // page].long(), :, t % page, :]


def run_greedy(m, ref, ctx, steps, seed):
    """Greedy decode from position ctx on both decoders; returns per-step records."""
    m.reset(ctx)
    tok = int(torch.randint(0, m.V, (1,), generator=torch.Generator().manual_seed(seed)))
    recs = []
    for k in range(steps):
        m.tok.fill_(tok)
        m.run_step()
        lg = m.logits.float().cpu()
        tg = int(m.tok)
        lr, tr = ref.step(tok, ctx + k)
        lr = lr.float()
        max_abs, max_rel = err(lg, lr)
        top2 = lr.topk(2).values
        recs.append({"step": k, "tok_in": tok, "gpu": tg, "ref": tr, "max_abs": max_abs, "max_rel": max_rel,
                     "margin": float(top2[0] - top2[1]), "gpu_argmax_matches_logits": tg == int(lg.argmax())})
        tok = tg
    return recs


def check(recs, m, ref, ctx, what):
    for r in recs:
        print(f"{what} step {r['step']}: max_rel {r['max_rel']:.2e} tokens gpu {r['gpu']} ref {r['ref']} "
              f"margin {r['margin']:.4f}", flush=True)
    for r in recs:
        assert np.isfinite(r["max_abs"]) and r["max_rel"] <= TOL, (what, r)
        assert r["gpu_argmax_matches_logits"], (what, r)   # the fused argmax picks the top logit it wrote
        if r["gpu"] != r["ref"]:
            assert r["margin"] <= 4 * r["max_abs"], (what, "greedy flip outside a near-tie", r)
    agree = sum(r["gpu"] == r["ref"] for r in recs)
    assert agree >= len(recs) - 2, (what, f"greedy agreement {agree}/{len(recs)}")
    steps = len(recs)
    mine = appended_rows(m.kv.cpu(), m.bt.cpu(), m.cfg.page, ctx, ctx + steps).float()
    theirs = appended_rows(ref.kv, ref.bt, ref.page, ctx, ctx + steps).float()
    _, kv_rel = err(mine, theirs)
    assert kv_rel <= TOL, (what, "appended K/V rows", kv_rel)


@pytest.fixture(scope="module")
def tinyllama():
    from runtime.model import DecodeConfig, Model
    from runtime.synth import TINYLLAMA, SyntheticLlama
    m = Model(SyntheticLlama(TINYLLAMA, seed=0), TINYLLAMA, DecodeConfig(lm_head="fp16", max_ctx=2048 + 64))
    w = oracle_weights(m)
    yield m, w, TINYLLAMA
    del m
    torch.cuda.empty_cache()


@pytest.mark.parametrize("ctx", [512, 2048])
def test_tinyllama_full_depth_against_oracle(tinyllama, ctx):
    """BASELINE config 4 at its own size: 22 layers, fp16 head, 16 greedy steps from context `ctx`."""
    m, w, shape = tinyllama
    steps = 16
    print(f"tinyllama full depth: ctx {ctx}, {steps} steps", flush=True)
    m.prepare(ctx + steps + 16)
    ref = RefDecoder(w, shape, max_ctx=m.cfg.max_ctx, page=m.cfg.page, block_table=m.bt.cpu(),
                     rope_theta=shape.rope_theta)
    fill_cache(m, ref, seed=ctx)
    check(run_greedy(m, ref, ctx, steps, seed=ctx + 1), m, ref, ctx, f"tinyllama ctx {ctx}")


def test_llama3_8b_full_depth_against_oracle():
    """BASELINE config 5 at its own size: 32 layers, head_dim 128, INT4 head, 6 greedy steps from context 4096."""
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LLAMA3_8B, SyntheticLlama
    ctx, steps = 4096, 6
    print(f"llama3-8b full depth: ctx {ctx}, {steps} steps", flush=True)
    m = Model(SyntheticLlama(LLAMA3_8B, seed=0), LLAMA3_8B, DecodeConfig(lm_head="int4", max_ctx=ctx + 32))
    m.prepare(ctx + steps + 16)
    ref = RefDecoder(oracle_weights(m), LLAMA3_8B, max_ctx=m.cfg.max_ctx, page=m.cfg.page, block_table=m.bt.cpu(),
                     rope_theta=LLAMA3_8B.rope_theta)
    fill_cache(m, ref, seed=8)
    check(run_greedy(m, ref, ctx, steps, seed=9), m, ref, ctx, f"llama3-8b ctx {ctx}")
    del m, ref
    torch.cuda.empty_cache()
