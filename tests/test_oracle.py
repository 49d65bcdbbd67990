"""CPU pins of the oracle (no GPU): every oracle function is checked against the reference's own known-answer tests,
hand-derived exact cases, brute force on tiny inputs, or an independent float64 computation, chosen so that a
plausible mistake (dropped term, wrong sign, wrong index or shift, transposed operand) fails at least one check.

Reference tests mirrored here: tests/test_quant_local.py:12-38 (pack KAT, roundtrip, RTN bound),
tests/test_ref_local.py:7-24 (split combine vs softmax, paged gather KAT), tests/test_kernels.py:48-68 (shape-1 closed
form and one-hot nibble sweep, applied to the oracle's dequantize + gemv).
"""
import math

import numpy as np
import pytest
import torch

from oracle import quant_ref as Q
from oracle import ref_ops as R
from oracle.decode_ref import RefDecoder


# ----------------------------------------------------------------------------------------------------------- format
def test_pack_known_word():
    """tests/test_quant_local.py:12-20: codes [0..7] pack to 0x75316420; (w >> 4i) & 0x000F000F = (2i, 2i+1)."""
    w = Q.pack(np.arange(8, dtype=np.uint8)[None])
    word = int(w.view(np.uint32)[0, 0])
    assert word == 0x75316420, hex(word)
    for i in range(4):
        t = (word >> (4 * i)) & 0x000F000F
        assert (t & 0xFFFF, t >> 16) == (2 * i, 2 * i + 1)


def test_pack_bit_positions_brute_force():
    """Every (element, value) pair lands at bits 4*(e//2) + 16*(e%2) and nowhere else."""
    for e in range(8):
        for v in range(16):
            q = np.zeros((1, 8), np.uint8)
            q[0, e] = v
            word = int(Q.pack(q).view(np.uint32)[0, 0])
            assert word == v << (4 * (e // 2) + 16 * (e % 2)), (e, v, hex(word))


def test_pack_unpack_roundtrip_and_bijection():
    """tests/test_quant_local.py:23-26 plus the reverse direction on random 32-bit words."""
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (64, 2048), dtype=np.uint8)
    assert np.array_equal(Q.unpack(Q.pack(q)), q)
    words = rng.integers(-2**31, 2**31, (16, 64), dtype=np.int64).astype(np.int32)
    assert np.array_equal(Q.pack(Q.unpack(words)), words)
    assert Q.pack(q).dtype == np.int32 and Q.pack(q).shape == (64, 256)


def test_pack_scale_zero_layout():
    s = np.array([[0.5, 0.25]], np.float16)
    z = np.array([[3, 7]], np.float16)
    sz = Q.pack_scale_zero(s, z)
    assert sz.shape == (1, 2, 2) and sz.dtype == np.float16
    assert sz.reshape(-1).tolist() == [0.5, 3.0, 0.25, 7.0]   # half2 (scale, zero) per group
    s2, z2 = Q.unpack_scale_zero(sz)
    assert np.array_equal(s2, s) and np.array_equal(z2, z)


def test_quantize_exact_ladder():
    """w = (k - 8) / 8: range 1.875 / 15 = 0.125 exactly, zero = 8, codes = k, dequant reproduces w exactly."""
    w = np.array([[(k - 8) / 8 for k in range(16)] * 2], np.float16)
    q, s, z = Q.quantize(w, 32)
    assert q[0].tolist() == list(range(16)) * 2
    assert float(s[0, 0]) == 0.125 and float(z[0, 0]) == 8.0
    assert np.array_equal(Q.dequantize(q, s, z, 32), w)


def test_quantize_round_half_even_ties():
    """Exact ties: scale 0.5 with w/scale in {0.5, 1.5, 2.5} and a zero-point tie -min/scale = 0.5.
    Round-half-to-even (torch.round) gives codes 1, 3, 3 and zero 0; round-half-up would give 2, 3, 4 and zero 1."""
    w = np.array([[-0.5, 7.0, 0.25, 0.75, 1.25, 0.0, 0.0, 0.0] * 4], np.float16)
    q, s, z = Q.quantize(w, 32)
    assert float(s[0, 0]) == 0.5 and float(z[0, 0]) == 1.0
    assert q[0, :8].tolist() == [0, 15, 1, 3, 3, 1, 1, 1]
    w = np.array([[-0.25, 7.25, 0, 0, 0, 0, 0, 0] * 4], np.float16)
    q, s, z = Q.quantize(w, 32)
    assert float(z[0, 0]) == 0.0 and q[0, :2].tolist() == [0, 14]


def test_quantize_degenerate_groups():
    """Constant group: range 0 -> scale floored at float32(1e-6), rounded to fp16 (17 * 2^-24); zero clamps."""
    q, s, z = Q.quantize(np.zeros((1, 32), np.float16), 32)
    assert float(s[0, 0]) == 17 * 2.0 ** -24 and float(z[0, 0]) == 0.0 and int(q.max()) == 0
    q, s, z = Q.quantize(np.full((1, 32), 0.7, np.float16), 32)
    assert float(z[0, 0]) == 0.0 and int(q.min()) == 15
    q, s, z = Q.quantize(np.full((1, 32), -0.7, np.float16), 32)
    assert float(z[0, 0]) == 15.0 and int(q.max()) == 0


def test_quantize_properties_random():
    """On random fp16 weights (G 32..256): scale is the fp16 nearest (max-min)/15; zero and codes are the nearest
    integers (up to clamping); RTN error <= scale/2 + fp16 rounding (tests/test_quant_local.py:29-38)."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float16)
    for g in (32, 64, 128, 256):
        q, s, z = Q.quantize(w, g)
        wf = w.astype(np.float64).reshape(64, -1, g)
        lo, hi = wf.min(-1), wf.max(-1)
        sf = s.astype(np.float64)
        ulp = np.spacing(np.abs(s).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(sf - (hi - lo) / 15) <= 0.5 * ulp * 1.0001 + 1e-12)
        zf = z.astype(np.float64)
        assert np.all(zf == np.round(zf)) and zf.min() >= 0 and zf.max() <= 15
        assert np.all((np.abs(zf - (-lo / sf)) <= 0.5 + 1e-6) | (zf == 0) | (zf == 15))
        t = wf / sf[..., None] + zf[..., None]
        qf = q.reshape(64, -1, g).astype(np.float64)
        assert np.all((np.abs(qf - t) <= 0.5 + 1e-5) | (qf == 0) | (qf == 15))
        err = np.abs(Q.dequantize(q, s, z, g).astype(np.float64) - w.astype(np.float64)).reshape(64, -1, g)
        assert np.all(err <= sf[..., None] * 0.5 + 2e-3 * np.abs(wf).max() + 1e-6)


def test_dequantize_single_rounding():
    """fp16((q - z) * s): (q - z) * s is exact in float64, so the oracle equals its float64 product rounded once."""
    rng = np.random.default_rng(2)
    q = rng.integers(0, 16, (8, 256), dtype=np.uint8)
    s = (rng.random((8, 2)) * 0.01 + 1e-4).astype(np.float16)
    z = rng.integers(0, 16, (8, 2)).astype(np.float16)
    exact = (q.astype(np.float64).reshape(8, 2, 128) - z.astype(np.float64)[..., None]) * s.astype(np.float64)[..., None]
    assert np.array_equal(Q.dequantize(q, s, z, 128), exact.reshape(8, 256).astype(np.float16))


@pytest.mark.parametrize("group", [32, 64, 128, 256])
def test_dequantize_packed_equals_unpack_then_dequantize(group):
    """The torch form bit for bit equals the numpy unpack + dequantize, on random words (every nibble value, negative
    int32 words, so the arithmetic shift of the sign bit is exercised) and on a real RTN quantization."""
    rng = np.random.default_rng(group)
    words = rng.integers(-2**31, 2**31, (24, 512 // 8), dtype=np.int64).astype(np.int32)
    s = (rng.random((24, 512 // group)) * 0.02 + 1e-5).astype(np.float16)
    z = rng.integers(0, 16, (24, 512 // group)).astype(np.float16)
    sz = Q.pack_scale_zero(s, z)
    want = Q.dequantize(Q.unpack(words), s, z, group)
    got = Q.dequantize_packed(torch.from_numpy(words), torch.from_numpy(sz), group).numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float16)
    q, s, z = Q.quantize(w, group)
    got = Q.dequantize_packed(torch.from_numpy(Q.pack(q)), torch.from_numpy(Q.pack_scale_zero(s, z)), group).numpy()
    assert np.array_equal(got.view(np.uint16), Q.dequantize(q, s, z, group).view(np.uint16))


def test_byte_counts_match_arrays_and_published_figures():
    """nbytes is the size of the packed words plus the scale/zero pairs the format produces; gemv_bytes adds x and y.
    Published figures: 6,142,976 B for the reference's 2048 x 5632 G128 down GEMV (RESULTS.md:204, the same bytes as
    BASELINE config 1) and 31,232,000 B at 4096 x 14336 G128."""
    rng = np.random.default_rng(5)
    for N, K, G in ((48, 256, 64), (8, 1024, 128), (16, 512, 256)):
        q, s, z = Q.quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float16), G)
        assert Q.nbytes(N, K, G) == Q.pack(q).nbytes + Q.pack_scale_zero(s, z).nbytes
        assert Q.gemv_bytes(N, K, G) == Q.nbytes(N, K, G) + 2 * K + 2 * N
    assert Q.gemv_bytes(2048, 5632, 128) == Q.gemv_bytes(5632, 2048, 128) == 6_142_976
    assert Q.gemv_bytes(4096, 14336, 128) == Q.gemv_bytes(14336, 4096, 128) == 31_232_000


def _shape1():
    """tests/test_kernels.py:47-56: q[r,k] = (k+r) % 16, zero 8, scale (r+1)/2, K = G = 128."""
    N, K = 4, 128
    q = np.array([[(k + r) % 16 for k in range(K)] for r in range(N)], np.uint8)
    s = np.array([[(r + 1) * 0.5] for r in range(N)], np.float16)
    z = np.full((N, 1), 8.0, np.float16)
    return q, s, z


def test_gemv_shape1_closed_form():
    """x = 1 -> y = [-32, -64, -96, -128] exactly; one-hot x_k -> y[r] = (q[r,k] - 8) * s[r] exactly."""
    q, s, z = _shape1()
    wref = torch.from_numpy(Q.dequantize(q, s, z, 128))
    y = R.gemv_ref(wref, torch.ones(128, dtype=torch.float16))
    assert y.tolist() == [-32.0, -64.0, -96.0, -128.0]
    for k in range(128):
        x = torch.zeros(128, dtype=torch.float16)
        x[k] = 1
        want = (q[:, k].astype(np.float64) - 8) * s[:, 0].astype(np.float64)
        assert R.gemv_ref(wref, x).double().numpy().tolist() == want.tolist()


def test_gemv_vs_float64():
    """Rectangular N != K so a transposed operand cannot pass; float64 matvec is the library routine."""
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(96, 320, generator=g) * 0.02).half()
    x = torch.randn(320, generator=g).half()
    y = R.gemv_ref(w, x)
    ref = (w.double() @ x.double())
    assert y.dtype == torch.float16 and y.shape == (96,)
    assert (y.double() - ref).abs().max() <= 1e-3 * ref.abs().max()


# ----------------------------------------------------------------------------------------------------- norm / act
def test_add_rmsnorm_residual_is_fp16_add():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(2048, generator=g) * 3).half()
    d = torch.randn(2048, generator=g).half()
    w = (1 + 0.1 * torch.randn(2048, generator=g)).half()
    xn, out = R.add_rmsnorm_ref(x, d, w, 1e-5)
    assert np.array_equal(xn.numpy(), x.numpy() + d.numpy())          # numpy fp16 add: one correct rounding
    xf = xn.double()
    h = (xf / torch.sqrt((xf * xf).mean() + 1e-5)).half()
    want = (w.double() * h.double())
    assert (out.double() - want).abs().max() <= 2 ** -10 * want.abs().max()
    xn2, out2 = R.add_rmsnorm_ref(x, None, w, 1e-5)
    assert xn2 is x


def test_add_rmsnorm_eps_known_answer():
    """Constant x = 2^-10: out = x / sqrt(x^2 + eps) = 0.295067 (eps 1e-5); without eps it would be 1.0."""
    x = torch.full((64,), 2.0 ** -10, dtype=torch.float16)
    _, out = R.add_rmsnorm_ref(x, None, torch.ones(64, dtype=torch.float16), 1e-5)
    want = 2.0 ** -10 / math.sqrt(2.0 ** -20 + 1e-5)
    assert abs(float(out[0]) - want) <= 2e-3 * want and abs(want - 0.295067) < 1e-5


def test_swiglu_known_answers():
    g = torch.tensor([0.0, 10.0, -10.0, 1.0], dtype=torch.float16)
    u = torch.tensor([3.0, 2.0, 5.0, 1.0], dtype=torch.float16)
    out = R.swiglu_ref(torch.cat([g, u]))
    silu1 = 1.0 / (1.0 + math.exp(-1.0))
    want = [0.0, 20.0, float(np.float16(-10.0 / (1 + math.exp(10.0)))) * 5.0, float(np.float16(silu1))]
    assert out.double().tolist() == pytest.approx(want, rel=1e-3, abs=1e-6)
    # gate and up are not interchangeable: silu(3)*0 != silu(0)*3
    assert float(R.swiglu_ref(torch.tensor([3.0, 0.0], dtype=torch.float16))[0]) == 0.0


def test_swiglu_vs_float64():
    g = torch.Generator().manual_seed(5)
    gu = (torch.randn(2 * 512, generator=g) * 2).half()
    gate, up = gu[:512].double(), gu[512:].double()
    s16 = (gate / (1 + torch.exp(-gate))).half().double()
    want = s16 * up
    assert (R.swiglu_ref(gu).double() - want).abs().max() <= 2 ** -10 * want.abs().max()


# ------------------------------------------------------------------------------------------------------------ rope
def test_rope_tables_closed_forms():
    cos, sin = R.rope_tables(4096, 64, 10000.0)
    assert cos.shape == (4096, 32) and cos.dtype == torch.float32
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    assert abs(float(cos[1, 0]) - math.cos(1.0)) < 1e-7                       # i = 0: frequency 1
    assert abs(float(cos[1, 1]) - 0.7317609758) < 1e-7                         # cos(10000^(-1/32)) = cos(0.7498942)
    assert abs(float(sin[3, 31]) - math.sin(3 * 10000 ** (-62 / 64))) < 1e-7
    a, b = 1234, 789
    lhs = cos[a + b].double()
    rhs = cos[a].double() * cos[b].double() - sin[a].double() * sin[b].double()
    assert (lhs - rhs).abs().max() < 1e-6
    c128, _ = R.rope_tables(16, 128, 500000.0)
    assert abs(float(c128[5, 10]) - math.cos(5 * 500000.0 ** (-20 / 128))) < 1e-7


def test_rope_rotation_pairs_and_sign():
    cos, sin = R.rope_tables(64, 64)
    x = torch.zeros(1, 64, dtype=torch.float16)
    x[0, 3] = 1.0                                  # pair (3, 35)
    out = R.rope_ref(x, cos, sin, 7).double()
    assert abs(out[0, 3] - cos[7, 3]) < 1e-3 and abs(out[0, 35] - sin[7, 3]) < 1e-3
    assert out[0, :3].abs().sum() == 0 and out[0, 36:].abs().sum() == 0
    x2 = torch.zeros(1, 64, dtype=torch.float16)
    x2[0, 35] = 1.0
    out2 = R.rope_ref(x2, cos, sin, 7).double()
    assert abs(out2[0, 3] + sin[7, 3]) < 1e-3 and abs(out2[0, 35] - cos[7, 3]) < 1e-3
    g = torch.Generator().manual_seed(6)
    xr = torch.randn(8, 64, generator=g).half()
    assert torch.equal(R.rope_ref(xr, cos, sin, 0), xr)   # position 0 is the identity, bit for bit


def test_rope_append_placement_and_v_copy():
    cos, sin = R.rope_tables(128, 64)
    n_q, n_kv, P = 4, 2, 16
    g = torch.Generator().manual_seed(7)
    kc = torch.zeros(12, n_kv, P, 64, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    bt = torch.randperm(12, generator=g).int()
    qkv = torch.randn((n_q + 2 * n_kv) * 64, generator=g).half()
    qr = R.rope_append_ref(qkv, cos, sin, 37, kc, vc, bt, n_q, n_kv, 64, P)
    page = int(bt[2])
    assert torch.equal(vc[page, :, 5], qkv[(n_q + n_kv) * 64:].view(n_kv, 64))
    assert torch.equal(kc[page, :, 5], R.rope_ref(qkv[n_q * 64:(n_q + n_kv) * 64].view(n_kv, 64), cos, sin, 37))
    assert torch.equal(qr, R.rope_ref(qkv[:n_q * 64].view(n_q, 64), cos, sin, 37))
    assert int((kc != 0).sum()) == int((kc[page, :, 5] != 0).sum())   # nothing else written


# ------------------------------------------------------------------------------------------------------- attention
def test_paged_gather_known_answer():
    """tests/test_ref_local.py:18-24: token 37 lives in logical page 2, offset 5."""
    g = torch.Generator().manual_seed(0)
    kc = torch.randn(12, 4, 16, 64, generator=g).half()
    vc = torch.randn(12, 4, 16, 64, generator=g).half()
    bt = torch.randperm(12, generator=g).int()
    k, v = R.gather_kv(kc, vc, bt, 70, 16)
    assert k.shape == (70, 4, 64)
    assert torch.equal(k[37], kc[bt[2], :, 5]) and torch.equal(v[37], vc[bt[2], :, 5])
    assert torch.equal(k[69], kc[bt[4], :, 5])


def _attn_f64(q, k, v):
    n_q, D = q.shape
    rep = n_q // k.shape[1]
    out = np.zeros((n_q, D))
    for h in range(n_q):
        kk = k[:, h // rep].double().numpy()
        vv = v[:, h // rep].double().numpy()
        s = kk @ q[h].double().numpy() / math.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out


@pytest.mark.parametrize("n_q,n_kv,D,ctx", [(32, 4, 64, 100), (8, 8, 64, 33), (16, 4, 128, 70), (4, 2, 64, 1)])
def test_attention_vs_float64(n_q, n_kv, D, ctx):
    g = torch.Generator().manual_seed(8)
    q = torch.randn(n_q, D, generator=g).half()
    k = (torch.randn(ctx, n_kv, D, generator=g) * 3).half()
    v = torch.randn(ctx, n_kv, D, generator=g).half()
    out = R.attention_contiguous_ref(q, k, v).double().numpy()
    want = _attn_f64(q, k, v)
    assert np.abs(out - want).max() <= 2e-3 * np.abs(want).max()


def test_attention_special_cases():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(4, 64, generator=g).half()
    v = torch.randn(1, 2, 64, generator=g).half()
    k = torch.randn(1, 2, 64, generator=g).half()
    out = R.attention_contiguous_ref(q, k, v)          # ctx = 1: softmax over one token returns v0 exactly
    assert torch.equal(out[0], v[0, 0]) and torch.equal(out[1], v[0, 0])
    assert torch.equal(out[2], v[0, 1]) and torch.equal(out[3], v[0, 1])   # GQA: heads 2,3 read kv head 1
    kk = torch.randn(10, 2, 64, generator=g).half()
    vv = torch.randn(10, 2, 64, generator=g).half()
    out0 = R.attention_contiguous_ref(torch.zeros(4, 64, dtype=torch.float16), kk, vv)   # q = 0: mean of V
    assert (out0[0].double() - vv[:, 0].double().mean(0)).abs().max() < 2e-3


def test_split_combine_matches_softmax():
    """tests/test_ref_local.py:7-16 grid: ctx x K-scale x part, tolerance 2e-3 absolute."""
    g = torch.Generator().manual_seed(0)
    for ctx in (1, 17, 128, 1000):
        for scale in (1.0, 8.0):
            q = torch.randn(32, 64, generator=g).half()
            k = (torch.randn(ctx, 4, 64, generator=g) * scale).half()
            v = torch.randn(ctx, 4, 64, generator=g).half()
            ref = R.attention_contiguous_ref(q, k, v)
            for part in (1, 16, 64, 100, 4096):
                out = R.split_softmax_combine_ref(q, k, v, part)
                assert (out.float() - ref.float()).abs().max().item() < 2e-3, (ctx, scale, part)


def test_paged_attention_equals_gather_then_attend():
    g = torch.Generator().manual_seed(10)
    kc = torch.randn(9, 4, 16, 64, generator=g).half()
    vc = torch.randn(9, 4, 16, 64, generator=g).half()
    bt = torch.randperm(9, generator=g).int()
    q = torch.randn(32, 64, generator=g).half()
    k, v = R.gather_kv(kc, vc, bt, 100, 16)
    assert torch.equal(R.paged_attention_ref(q, kc, vc, bt, 100, 16), R.attention_contiguous_ref(q, k, v))


# ---------------------------------------------------------------------------------------------------- decode step
class _Shape:
    hidden_size, num_hidden_layers, num_attention_heads, num_key_value_heads = 128, 2, 4, 2
    intermediate_size, vocab_size, rms_norm_eps = 256, 64, 1e-5


def _f64_llama_logits(w, shape, tokens, theta=10000.0):
    """Independent float64 Llama forward over the whole prefix (contiguous KV, no paging, no fp16 rounding):
    pins the composition order (pre-norm residual blocks, fused qkv/gu split, GQA, final norm, head)."""
    H, nq, nkv = shape.hidden_size, shape.num_attention_heads, shape.num_key_value_heads
    D, I = H // nq, shape.intermediate_size
    dd = lambda t: t.double()

    def rms(x, wt):
        return dd(wt) * x / torch.sqrt((x * x).mean(-1, keepdim=True) + shape.rms_norm_eps)

    T = len(tokens)
    x = dd(w["emb"][torch.tensor(tokens)])
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.arange(T, dtype=torch.float64)[:, None] * inv[None]
    c, s = torch.cos(ang), torch.sin(ang)

    def rot(t):                                   # t [T, heads, D]
        a, b = t[..., :D // 2], t[..., D // 2:]
        return torch.cat([a * c[:, None] - b * s[:, None], b * c[:, None] + a * s[:, None]], -1)

    for lw in w["layers"]:
        h = rms(x, lw["ln1"]) @ dd(lw["qkv"]).T
        q = rot(h[:, :nq * D].view(T, nq, D))
        k = rot(h[:, nq * D:(nq + nkv) * D].view(T, nkv, D))
        v = h[:, (nq + nkv) * D:].view(T, nkv, D)
        att = torch.zeros(T, nq, D, dtype=torch.float64)
        for hh in range(nq):
            sc = q[:, hh] @ k[:, hh // (nq // nkv)].T / math.sqrt(D)
            sc = sc + torch.triu(torch.full((T, T), float("-inf"), dtype=torch.float64), 1)
            att[:, hh] = torch.softmax(sc, -1) @ v[:, hh // (nq // nkv)]
        x = x + att.reshape(T, -1) @ dd(lw["o"]).T
        gu = rms(x, lw["ln2"]) @ dd(lw["gu"]).T
        x = x + (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]) @ dd(lw["down"]).T
    return rms(x, w["norm_f"]) @ dd(w["lm_head"]).T


def test_decode_ref_matches_float64_llama():
    sh = _Shape
    g = torch.Generator().manual_seed(11)
    H, I, V = sh.hidden_size, sh.intermediate_size, sh.vocab_size
    D = H // sh.num_attention_heads
    qkv_rows = (sh.num_attention_heads + 2 * sh.num_key_value_heads) * D
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).half()
    w = {"emb": mk(V, H), "norm_f": (1 + 0.1 * torch.randn(H, generator=g)).half(), "lm_head": mk(V, H),
         "layers": [{"ln1": (1 + 0.1 * torch.randn(H, generator=g)).half(),
                     "ln2": (1 + 0.1 * torch.randn(H, generator=g)).half(),
                     "qkv": mk(qkv_rows, H), "o": mk(H, H), "gu": mk(2 * I, H), "down": mk(H, I)}
                    for _ in range(sh.num_hidden_layers)]}
    bt = torch.randperm(5, generator=g).int()
    dec = RefDecoder(w, sh, max_ctx=64, page=16, block_table=bt)
    tokens = [3, 17, 60, 5, 41, 22, 9, 33, 1, 50, 7, 28, 44, 12, 36, 19, 58, 2]
    want = _f64_llama_logits(w, sh, tokens)
    for pos, t in enumerate(tokens):
        logits, _ = dec.step(t, pos)
        err = (logits.double() - want[pos]).abs().max()
        assert err <= 2e-2 * want[pos].abs().max(), (pos, float(err))


def test_decode_ref_batched_steps_equal_sequential_steps():
    """RefDecoder.steps (T teacher-forced steps in one pass) is T calls of RefDecoder.step: same logits up to the fp32
    summation order of the products, same greedy tokens, same cache rows; also from a pre-filled cache (pos0 > 0)."""
    sh = _Shape
    g = torch.Generator().manual_seed(12)
    H, I, V = sh.hidden_size, sh.intermediate_size, sh.vocab_size
    D = H // sh.num_attention_heads
    qkv_rows = (sh.num_attention_heads + 2 * sh.num_key_value_heads) * D
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).half()
    w = {"emb": mk(V, H), "norm_f": (1 + 0.1 * torch.randn(H, generator=g)).half(), "lm_head": mk(V, H),
         "layers": [{"ln1": (1 + 0.1 * torch.randn(H, generator=g)).half(),
                     "ln2": (1 + 0.1 * torch.randn(H, generator=g)).half(),
                     "qkv": mk(qkv_rows, H), "o": mk(H, H), "gu": mk(2 * I, H), "down": mk(H, I)}
                    for _ in range(sh.num_hidden_layers)]}
    bt = torch.randperm(5, generator=g).int()
    tokens = [3, 17, 60, 5, 41, 22, 9, 33, 1, 50, 7, 28, 44, 12, 36, 19, 58, 2, 11, 40]
    seq = RefDecoder(w, sh, max_ctx=64, page=16, block_table=bt)
    want = [seq.step(t, p) for p, t in enumerate(tokens)]
    for split in (0, 7):                                   # all rows at once; 7 sequential steps then a batch
        bat = RefDecoder(w, sh, max_ctx=64, page=16, block_table=bt)
        for p in range(split):
            bat.step(tokens[p], p)
        logits, top = bat.steps(tokens[split:], split)
        for r, (lw, tw) in enumerate(want[split:]):
            d = (logits[r].float() - lw.float()).abs().max()
            assert d <= 2e-3 * lw.float().abs().max(), (split, r, float(d))
            margin = lw.float().topk(2).values
            assert int(top[r]) == tw or float(margin[0] - margin[1]) <= 2 * float(d), (split, r)
        d = (bat.kv.float() - seq.kv.float()).abs().max()
        assert d <= 2e-3 * seq.kv.float().abs().max(), float(d)
