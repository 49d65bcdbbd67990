"""Full-depth decode parity: the graph-captured HIP decode step of the BASELINE models at their real size against the
CPU oracle decoder (oracle/decode_ref.py, the reference's backend="ref" composition, runtime/model.py:216-233).

  * config 4 as BASELINE states it: TinyLlama-1.1B architecture (22 layers, hidden 2048, 32 q / 4 kv heads, head_dim
    64, SwiGLU 5632, vocab 32000), INT4 G128 body, fp16 LM head; a random-token prompt of 512 or 2048 tokens
    teacher-forced through the decode graph (the reference's prompt path, runtime/model.py:278-286), then 256 greedy
    tokens. The oracle runs the same prompt and the GPU's greedy tokens as teacher-forced batched steps
    (RefDecoder.steps: the step composition applied to every row, pinned against RefDecoder.step), with its own
    K/V cache, so both decoders build their whole context independently;
  * config 5: Llama-3-8B architecture (32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 14336,
    vocab 128256, rope theta 5e5), INT4 G128 body and LM head, context 4096, 32 greedy steps. Its 4096-token prompt
    would cost the CPU oracle minutes, so positions 0 .. 4095 of every layer's K and V cache start from the same
    seeded N(0, 1) values in both decoders.

The oracle's weights are the model's INT4 codes dequantized by the oracle (quant_ref.dequantize_packed, pinned
bit-exact to the numpy restatement on the CPU; here it runs on the GPU's tensors so that the 8B model's 7.5 G weights
dequantize in seconds, and a sampled block of rows is checked against the numpy path) and held as float32 copies of
their fp16 values on the CPU.

Bars (the reference's, tests/test_kernels.py and tests/test_runtime_local.py:21-28):
  * logits of every compared step within 2e-2 normwise (the whole-step bar of the golden decode test);
  * greedy agreement: the GPU's argmax equals the oracle's, except where the oracle's top1 - top2 margin is within
    4x that step's largest logit difference (a near-tie the observed error can flip); every flip is printed with its
    margin, and the agreement is reported (bench/e2e.py:180-203 reports it the same way);
  * the K and V rows of every position the decoders wrote within 2e-2 normwise of the oracle's.
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


def greedy_on_gpu(m, ctx, steps, seed):
    """Greedy decode on the GPU from position ctx, the cache below ctx as it is: the input of step k is the GPU's own
    choice from step k - 1 (a seeded random token for k = 0). Returns (inputs [steps], logits fp32 [steps, V],
    chosen tokens [steps])."""
    m.reset(ctx)
    tok = int(torch.randint(0, m.V, (1,), generator=torch.Generator().manual_seed(seed)))
    m.tok.fill_(tok)
    inputs, rows, picks = [], [], []
    for _ in range(steps):
        inputs.append(m.tok.clone())
        m.run_step()
        rows.append(m.logits.clone())
        picks.append(m.tok.clone())
    return torch.cat(inputs).cpu(), torch.stack(rows).float().cpu(), torch.cat(picks).cpu()


def oracle_steps(ref, tokens, pos0, keep_from, chunk=512):
    """The oracle's teacher-forced steps over tokens at positions pos0 .. (chunks of `chunk` rows); returns the logits
    (fp32) and argmax of the rows at positions >= keep_from."""
    lg, top = [], []
    for c in range(0, len(tokens), chunk):
        l, t = ref.steps(tokens[c:c + chunk], pos0 + c)
        lo = max(0, keep_from - (pos0 + c))
        lg.append(l[lo:].float())
        top.append(t[lo:])
    return torch.cat(lg), torch.cat(top)


def records(gpu_logits, gpu_tok, ref_logits, ref_tok):
    recs = []
    for k in range(gpu_logits.shape[0]):
        max_abs, max_rel = err(gpu_logits[k], ref_logits[k])
        top2 = ref_logits[k].topk(2).values
        recs.append({"step": k, "gpu": int(gpu_tok[k]), "ref": int(ref_tok[k]), "max_abs": max_abs,
                     "max_rel": max_rel, "margin": float(top2[0] - top2[1]),
                     "gpu_argmax_matches_logits": int(gpu_tok[k]) == int(gpu_logits[k].argmax())})
    return recs


def check(recs, m, ref, lo, hi, what, min_agree=0.9):
    worst = max(r["max_rel"] for r in recs)
    flips = [r for r in recs if r["gpu"] != r["ref"]]
    agree = len(recs) - len(flips)
    print(f"{what}: {len(recs)} steps, logits max_rel <= {worst:.2e}, greedy agreement {agree}/{len(recs)}",
          flush=True)
    for r in flips:
        print(f"{what} flip at step {r['step']}: gpu {r['gpu']} ref {r['ref']} margin {r['margin']:.4f} "
              f"(max |dlogit| {r['max_abs']:.4f})", flush=True)
    for r in recs:
        assert np.isfinite(r["max_abs"]) and r["max_rel"] <= TOL, (what, r)
        assert r["gpu_argmax_matches_logits"], (what, r)   # the fused argmax picks the top logit it wrote
        if r["gpu"] != r["ref"]:
            assert r["margin"] <= 4 * r["max_abs"], (what, "greedy flip outside a near-tie", r)
    assert agree >= min_agree * len(recs), (what, f"greedy agreement {agree}/{len(recs)}")
    mine = appended_rows(m.kv.cpu(), m.bt.cpu(), m.cfg.page, lo, hi).float()
    theirs = appended_rows(ref.kv, ref.bt, ref.page, lo, hi).float()
    _, kv_rel = err(mine, theirs)
    print(f"{what}: K/V rows {lo}..{hi - 1} max_rel {kv_rel:.2e}", flush=True)
    assert kv_rel <= TOL, (what, "K/V rows", kv_rel)


@pytest.fixture(scope="module")
def tinyllama():
    from runtime.model import DecodeConfig, Model
    from runtime.synth import TINYLLAMA, SyntheticLlama
    m = Model(SyntheticLlama(TINYLLAMA, seed=0), TINYLLAMA, DecodeConfig(lm_head="fp16", max_ctx=2048 + 256 + 16))
    w = oracle_weights(m)
    yield m, w, TINYLLAMA
    del m
    torch.cuda.empty_cache()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("ctx", [512, 2048])
def test_tinyllama_full_depth_against_oracle(tinyllama, ctx):
    """BASELINE config 4 as stated: 22 layers, fp16 head, a random-token prompt of `ctx` tokens, then 256 greedy
    tokens; compared: the prompt's last step and every greedy step."""
    m, w, shape = tinyllama
    new = 256
    print(f"tinyllama full depth: {ctx}-token prompt, {new} greedy tokens", flush=True)
    m.prepare(ctx + new + 1)
    prompt = torch.randint(0, m.V, (ctx,), generator=torch.Generator().manual_seed(ctx))
    m.reset(0)
    m.teacher_force(prompt)
    rows, picks = [m.logits.clone()], [m.tok.clone()]
    for _ in range(new - 1):
        m.run_step()
        rows.append(m.logits.clone())
        picks.append(m.tok.clone())
    gpu_logits, gpu_tok = torch.stack(rows).float().cpu(), torch.cat(picks).cpu()
    ref = RefDecoder(w, shape, max_ctx=m.cfg.max_ctx, page=m.cfg.page, block_table=m.bt.cpu(),
                     rope_theta=shape.rope_theta)
    tokens = torch.cat([prompt, gpu_tok[:-1]])        # the prompt, then the GPU's greedy tokens as inputs
    ref_logits, ref_tok = oracle_steps(ref, tokens, 0, keep_from=ctx - 1)
    check(records(gpu_logits, gpu_tok, ref_logits, ref_tok), m, ref, 0, ctx + new - 1, f"tinyllama ctx {ctx}")


@pytest.mark.timeout(900)
def test_llama3_8b_full_depth_against_oracle():
    """BASELINE config 5 at its own size: 32 layers, head_dim 128, INT4 head, 32 greedy steps from context 4096 (the
    cache below it seeded identically in both decoders)."""
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LLAMA3_8B, SyntheticLlama
    ctx, steps = 4096, 32
    print(f"llama3-8b full depth: ctx {ctx}, {steps} steps", flush=True)
    m = Model(SyntheticLlama(LLAMA3_8B, seed=0), LLAMA3_8B, DecodeConfig(lm_head="int4", max_ctx=ctx + 48))
    m.prepare(ctx + steps + 16)
    ref = RefDecoder(oracle_weights(m), LLAMA3_8B, max_ctx=m.cfg.max_ctx, page=m.cfg.page, block_table=m.bt.cpu(),
                     rope_theta=LLAMA3_8B.rope_theta)
    fill_cache(m, ref, seed=8)
    inputs, gpu_logits, gpu_tok = greedy_on_gpu(m, ctx, steps, seed=9)
    ref_logits, ref_tok = oracle_steps(ref, inputs, ctx, keep_from=ctx)
    check(records(gpu_logits, gpu_tok, ref_logits, ref_tok), m, ref, ctx, ctx + steps, f"llama3-8b ctx {ctx}")
    del m, ref
    torch.cuda.empty_cache()
