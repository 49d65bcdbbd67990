"""GPU checks of the calibration producers: the HIP range-clipping quantizer (dk_quantize_w4 clip=1) against the
reference's own clip outputs and the oracle's clip search, and decode steps of models built from clipped and from
GPTQ-precomputed codes (DecodeConfig quant "clip" / "pre") against the oracle decoder on the same dequantized weights.
The clip choice is an argmin over summed errors: where two factors' errors agree to float32 summation noise the GPU
(fp64 sums) and the oracle (fp64 sums, another order) may pick differently, so such groups are checked to be
near-ties instead of equal."""
import pathlib

import numpy as np
import pytest
import torch

from helpers import DEV, gen
from oracle import quant_ref as Q

pytestmark = pytest.mark.gpu

GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "quant_calib.npz")


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


def gpu_clip(K, w, G):
    N, Kd = w.shape
    packed = torch.empty(N, Kd // 8, dtype=torch.int32, device=DEV)
    sz = torch.empty(N, Kd // G, 2, dtype=torch.half, device=DEV)
    K.quantize_w4(torch.as_tensor(w).to(DEV), packed, sz, G, clip=True)
    return packed.cpu().numpy(), sz.cpu().numpy()


@pytest.mark.parametrize("G", (64, 128))
def test_gpu_clip_matches_reference(K, G):
    packed, sz = gpu_clip(K, GOLD["w"], G)
    assert np.array_equal(packed, Q.pack(GOLD[f"clip{G}_q"]))
    assert np.array_equal(sz.view(np.uint16), Q.pack_scale_zero(GOLD[f"clip{G}_s"], GOLD[f"clip{G}_z"]).view(np.uint16))


@pytest.mark.parametrize("N,Kd,G", [(256, 4096, 32), (256, 4096, 128), (100, 2048, 256), (64, 1024, 512),
                                    (5632, 2048, 128)])
def test_gpu_clip_matches_oracle(K, N, Kd, G):
    g = gen(N + Kd + G)
    w = torch.randn(N, Kd, generator=g) * 0.02
    w[torch.rand(N, Kd, generator=g) < 0.005] *= 8
    w = w.half().numpy()
    packed, sz = gpu_clip(K, w, G)
    q, s, z = Q.quantize(w, G, clip=True)
    ref_sz = Q.pack_scale_zero(s, z)
    diff = np.any(sz.view(np.uint16) != ref_sz.view(np.uint16), axis=-1)       # [N, K/G] groups that differ
    assert diff.sum() <= max(1, diff.size // 10000), f"{diff.sum()} of {diff.size} groups differ"
    if diff.any():                                                            # each must be a near-tie
        wf = w.astype(np.float32).reshape(N, Kd // G, G)
        sg, zg = sz[..., 0].astype(np.float32)[..., None], sz[..., 1].astype(np.float32)[..., None]
        eg = Q.clip_errors(wf, sg, zg)[..., 0]
        eo = Q.clip_errors(wf, s.astype(np.float32)[..., None], z.astype(np.float32)[..., None])[..., 0]
        assert np.all(np.abs(eg[diff] - eo[diff]) <= 1e-6 * eo[diff]), (eg[diff], eo[diff])
    ok_rows = ~diff.any(axis=1)
    assert np.array_equal(packed[ok_rows], Q.pack(q)[ok_rows])


def _decode_against_oracle(m, shape, tokens=(5, 17, 99, 3)):
    from __graft_entry__ import _ref_weights
    from oracle.decode_ref import RefDecoder
    ref = RefDecoder(_ref_weights(m, shape), shape, max_ctx=64, page=16, block_table=m.bt.cpu())
    m.reset(0)
    for p, t in enumerate(tokens):
        m.tok.fill_(t)
        m.run_step()
        lr, _ = ref.step(t, p)
        e = ((m.logits.float().cpu() - lr.float()).abs().max() / lr.float().abs().max()).item()
        assert e <= 2e-2, f"step {p}: logits max_rel {e}"


def test_decode_with_clipped_weights(K):
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(256, 2, 4, 2, 512, 1000)
    sd = SyntheticLlama(shape, seed=2, device=DEV, std=0.05)
    m = Model(sd, shape, DecodeConfig(max_ctx=64, device=DEV, quant="clip"))
    m.prepare(64)
    # the model's packed codes are the clip producer's
    lw = m.layers[0]["o"]
    w = sd["model.layers.0.self_attn.o_proj.weight"].cpu()
    q, s, z = Q.quantize(w.numpy(), 128, clip=True)
    assert np.array_equal(lw.packed.cpu().numpy(), Q.pack(q))
    _decode_against_oracle(m, shape)


def test_decode_with_gptq_codes(K):
    """runtime.gptq.calibrate on an HF Llama holding the synthetic weights (CPU), then a decode runtime built from the
    precomputed codes: its packed weights are exactly the codes, and its steps match the oracle decoder."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from runtime import gptq
    from runtime.model import DecodeConfig, Model
    from runtime.quant import pack_codes
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(256, 2, 4, 2, 512, 1000)
    sd = {k: v for k, v in SyntheticLlama(shape, seed=3, device="cpu", std=0.05).items()}
    hf = LlamaForCausalLM(LlamaConfig(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                                      rms_norm_eps=1e-5, rope_theta=10000.0)).eval()
    hf.load_state_dict({k: v.float() for k, v in sd.items()})
    qp = gptq.calibrate(hf, gptq.random_windows(1000, n=8, L=48), group=128, log=lambda *a: None)
    m = Model(sd, shape, DecodeConfig(max_ctx=64, device=DEV, quant="pre", qparams=qp, lm_head="int4"))
    m.prepare(64)
    packed, _ = pack_codes(*qp["layers.1.down"])
    assert torch.equal(m.layers[1]["down"].packed.cpu(), packed)
    assert torch.equal(m.lm_head.packed.cpu(), pack_codes(*qp["lm_head"])[0])
    _decode_against_oracle(m, shape)
