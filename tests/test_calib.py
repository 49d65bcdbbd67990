"""CPU checks of the calibration producers (range clipping, GPTQ, the calibration driver) and of the oracle's clip
search. Pins: the reference's own outputs (tests/golden/quant_calib.npz, written by tests/golden/make_golden.py from
the reference's runtime/quant.py), and what the mathematics fixes -- the clip choice is the argmin of the group error
over the grid, GPTQ with a diagonal Hessian has no error feedback and is RTN exactly, GPTQ lowers the layer-output
error on correlated inputs (the reference's tests/test_quant_local.py:41-60)."""
import sys
import pathlib

import numpy as np
import pytest
import torch

from oracle import quant_ref as Q
from runtime import quant as RQ

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent / "golden"))
from make_golden import calib_hessian  # noqa: E402  (the fixture's own input recipe)

GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "quant_calib.npz")


def _bits(a):
    return np.asarray(a).view(np.uint16)


@pytest.mark.parametrize("G", (64, 128))
def test_oracle_clip_matches_reference(G):
    q, s, z = Q.quantize(GOLD["w"], G, clip=True)
    assert np.array_equal(q, GOLD[f"clip{G}_q"])
    assert np.array_equal(_bits(s), _bits(GOLD[f"clip{G}_s"])) and np.array_equal(_bits(z), _bits(GOLD[f"clip{G}_z"]))


@pytest.mark.parametrize("G", (64, 128))
def test_runtime_clip_params_match_reference(G):
    """runtime.quant.group_params(clip=True), the search GPTQ runs on its error-updated weights, on the CPU."""
    w = torch.from_numpy(GOLD["w"]).float()
    N, K = w.shape
    s, z = RQ.group_params(w.reshape(N, K // G, G), clip=True)
    assert np.array_equal(_bits(s.reshape(N, -1).half().numpy()), _bits(GOLD[f"clip{G}_s"]))
    assert np.array_equal(z.reshape(N, -1).half().numpy(), GOLD[f"clip{G}_z"])


def test_clip_choice_is_the_grid_argmin():
    """For every group the chosen (scale, zero) has the smallest float64 error over the seven factors, computed
    independently here, and never more than RTN's."""
    g = np.random.default_rng(3)
    w = (g.standard_normal((64, 512)) * 0.02).astype(np.float32)
    w[g.random(w.shape) < 0.01] *= 10
    G = 128
    wf = w.reshape(64, 4, G)
    s, z = Q.group_params(wf, clip=True)
    chosen = Q.clip_errors(wf, s, z)[..., 0]
    errs = []
    for a in Q.CLIP_GRID:
        lo, hi = wf.min(-1, keepdims=True) * np.float32(a), wf.max(-1, keepdims=True) * np.float32(a)
        st = np.maximum((hi - lo) / np.float32(15), np.float32(1e-6)).astype(np.float16).astype(np.float32)
        zt = np.clip(np.rint(-lo / st), 0, 15).astype(np.float32)
        d = ((np.clip(np.rint(wf / st) + zt, 0, 15) - zt) * st - wf).astype(np.float32)
        errs.append((d * d).astype(np.float64).sum(-1))     # squares in float32, as the reference squares
    errs = np.stack(errs)
    assert np.array_equal(chosen, errs.min(0))
    assert np.all(chosen <= errs[0])                         # never worse than RTN (factor 1.0)
    assert np.any(chosen < errs[0] * 0.99)                   # and the outliers make it matter


@pytest.mark.parametrize("tag,clip", (("gptq64", False), ("gptqclip64", True)))
def test_gptq_matches_reference(tag, clip):
    w = torch.from_numpy(GOLD["w"])
    H = calib_hessian(torch.from_numpy(GOLD["A"]), torch.from_numpy(GOLD["B"]))
    q, s, z = RQ.quantize_gptq(w, H, 64, clip=clip)
    assert torch.equal(q, torch.from_numpy(GOLD[f"{tag}_q"]))
    assert np.array_equal(_bits(s.numpy()), _bits(GOLD[f"{tag}_s"])) and torch.equal(z, torch.from_numpy(GOLD[f"{tag}_z"]))


@pytest.mark.parametrize("clip", (False, True))
def test_gptq_with_diagonal_hessian_is_rtn(clip):
    """H diagonal -> the upper Cholesky factor of H^-1 is diagonal, no rounding error reaches another column, and the
    codes are RTN's (clip: the clip search's), bit for bit."""
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(40, 256, generator=g) * 0.02).half()
    H = torch.diag(torch.rand(256, generator=g) + 0.1)
    q, s, z = RQ.quantize_gptq(w, H, 64, clip=clip)
    qr, sr, zr = Q.quantize(w.numpy(), 64, clip=clip)
    assert np.array_equal(q.numpy(), qr)
    assert np.array_equal(_bits(s.numpy()), _bits(sr)) and np.array_equal(z.numpy(), zr)


def test_gptq_and_clip_beat_rtn():
    """The reference's property test: clipping lowers the weight error, GPTQ lowers the output error (what it
    minimises) by more than 30%, and both stay in the kernel's format."""
    w = torch.from_numpy(GOLD["w"])
    A, B = torch.from_numpy(GOLD["A"]), torch.from_numpy(GOLD["B"])
    X = A @ B
    X[:, :8] *= 10
    H = calib_hessian(A, B)
    G = 64
    deq = lambda q, s, z: torch.from_numpy(Q.dequantize(np.asarray(q), np.asarray(s), np.asarray(z), G)).float()
    out_err = lambda *a: (X @ (deq(*a) - w.float()).t()).pow(2).mean().item()
    w_err = lambda *a: (deq(*a) - w.float()).pow(2).mean().item()
    rtn, clip = Q.quantize(w.numpy(), G), Q.quantize(w.numpy(), G, clip=True)
    gptq = tuple(t.numpy() for t in RQ.quantize_gptq(w, H, G))
    assert w_err(*clip) < w_err(*rtn)
    assert out_err(*gptq) < 0.7 * out_err(*rtn)
    for q, s, z in (clip, gptq):
        assert q.dtype == np.uint8 and int(q.max()) <= 15
        zf = z.astype(np.float32)
        assert np.array_equal(zf, np.round(zf)) and zf.min() >= 0 and zf.max() <= 15


def test_pack_codes_matches_oracle():
    g = np.random.default_rng(5)
    q = g.integers(0, 16, (24, 256), dtype=np.uint8)
    s = (g.random((24, 4)) * 0.01 + 1e-3).astype(np.float16)
    z = g.integers(0, 16, (24, 4)).astype(np.float16)
    packed, sz = RQ.pack_codes(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z))
    assert np.array_equal(packed.numpy(), Q.pack(q))
    assert np.array_equal(_bits(sz.numpy()), _bits(Q.pack_scale_zero(s, z)))


def _tiny_hf_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    return LlamaForCausalLM(cfg).eval()


def test_calibrate_tiny_hf_llama():
    """End-to-end mechanics of runtime.gptq.calibrate (as the reference's tests/test_quant_local.py:63-80): every
    projection and the head produced with the runtime's keys and shapes, codes in format, and the HF model's weights
    restored afterwards."""
    from runtime import gptq
    m = _tiny_hf_llama()
    before = {k: v.clone() for k, v in m.state_dict().items()}
    out = gptq.calibrate(m, gptq.random_windows(256, n=6, L=32), group=64, log=lambda *a: None)
    assert set(out) == {f"layers.{i}.{k}" for i in range(2) for k in ("qkv", "o", "gu", "down")} | {"lm_head"}
    assert out["layers.0.qkv"][0].shape == (128 + 2 * 64, 128) and out["layers.1.gu"][0].shape == (512, 128)
    assert out["layers.0.down"][0].shape == (128, 256) and out["lm_head"][1].shape == (256, 2)
    for q, s, z in out.values():
        assert q.dtype == torch.uint8 and int(q.max()) <= 15 and torch.equal(z.float(), z.float().round())
    assert all(torch.equal(before[k], v) for k, v in m.state_dict().items())


def test_calibrate_lowers_layer_output_error():
    """The calibration minimises what GPTQ is meant to: on the inputs the calibration itself saw, layer 0's qkv
    projection with the calibrated codes has a lower output error than with RTN codes (a wrong Hessian, e.g. from
    the wrong module's input or a transposed accumulation, fails this)."""
    from runtime import gptq
    m = _tiny_hf_llama(seed=1)
    wins = gptq.random_windows(256, n=8, L=32, seed=3)
    out = gptq.calibrate(m, wins, group=64, log=lambda *a: None)
    inputs = gptq._LayerInputs(m, wins)
    layer = m.model.layers[0]
    X = torch.cat([layer.input_layernorm(x).reshape(-1, 128) for x in inputs.states]).float()
    W = torch.cat([layer.self_attn.q_proj.weight, layer.self_attn.k_proj.weight, layer.self_attn.v_proj.weight]).float()
    deq = lambda q, s, z: torch.from_numpy(Q.dequantize(np.asarray(q), np.asarray(s), np.asarray(z), 64)).float()
    err = lambda wq: (X @ (wq - W).t()).pow(2).mean().item()
    e_gptq = err(deq(*out["layers.0.qkv"]))
    e_rtn = err(deq(*Q.quantize(W.detach().numpy(), 64)))
    assert e_gptq < 0.9 * e_rtn, (e_gptq, e_rtn)
