"""Decode-step parity of the model variants the runtime offers, against the CPU oracle decoder (oracle/decode_ref.py,
the reference's backend="ref" composition, runtime/model.py:216-233) with the bars of the full-depth test (logits
2e-2 normwise every step, greedy agreement outside near-ties, appended K/V rows 2e-2):

  * group sizes 64 and 256 (the reference's G knob, runtime/quant.py and tests/test_kernels.py), INT4 and fp16 LM
    heads, page 32, fp16 weights throughout, the attention combine as a launch instead of merged into the o
    projection, at TinyLlama widths (hidden 2048, 32 q / 4 kv heads, SwiGLU 5632) over 3 layers;
  * head_dim 128 (Llama-3-8B widths: hidden 4096, 32 q / 8 kv heads, SwiGLU 14336) with G64 and an INT4 head over
    2 layers;
  * long contexts (4000 and 12000 at TinyLlama widths, 8000 at head_dim 128), where the attention policy's later
    split bands run and the combine is a launch of its own.

Each case starts both decoders from the same seeded K/V cache at its context and steps 32 greedy tokens (the oracle
runs the GPU's greedy tokens as one batch of teacher-forced steps)."""
import pytest
import torch

from test_full_depth_gpu import check, fill_cache, greedy_on_gpu, oracle_steps, oracle_weights, records

pytestmark = pytest.mark.gpu
DEV = "cuda"

TINY_W = (2048, 3, 32, 4, 5632, 32000)
L3_W = (4096, 2, 32, 8, 14336, 32000)
# (name, widths, DecodeConfig overrides, ctx)
CASES = [("G64 int4 head", TINY_W, dict(group=64, lm_head="int4"), 300),
         ("G256 fp16 head page 32", TINY_W, dict(group=256, lm_head="fp16", page=32), 700),
         ("fp16 weights", TINY_W, dict(weights="fp16"), 400),
         ("combine launch", TINY_W, dict(combine_in_o=False), 512),
         ("D128 G64 int4 head", L3_W, dict(group=64, lm_head="int4"), 1000),
         # long contexts: the attention policy's later bands (more splits than the o projection merges, so the
         # combine runs as a launch) inside the whole step
         ("long ctx 4000", TINY_W, {}, 4000),
         ("long ctx 12000", TINY_W, {}, 12000),
         ("D128 long ctx 8000", L3_W, dict(group=64, lm_head="int4"), 8000)]


@pytest.mark.parametrize("name,widths,over,ctx", CASES, ids=[c[0] for c in CASES])
def test_decode_variant_against_oracle(name, widths, over, ctx):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from oracle.decode_ref import RefDecoder
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(*widths)
    steps = 32
    print(f"decode variant {name}: ctx {ctx}", flush=True)
    m = Model(SyntheticLlama(shape, seed=len(name)), shape, DecodeConfig(max_ctx=ctx + 64, device=DEV, **over))
    m.prepare(ctx + steps + 16)
    ref = RefDecoder(oracle_weights(m), shape, max_ctx=m.cfg.max_ctx, page=m.cfg.page, block_table=m.bt.cpu(),
                     rope_theta=shape.rope_theta)
    fill_cache(m, ref, seed=ctx + 1)
    inputs, gpu_logits, gpu_tok = greedy_on_gpu(m, ctx, steps, seed=ctx + 2)
    ref_logits, ref_tok = oracle_steps(ref, inputs, ctx, keep_from=ctx)
    check(records(gpu_logits, gpu_tok, ref_logits, ref_tok), m, ref, ctx, ctx + steps, name)
    del m, ref
    torch.cuda.empty_cache()
