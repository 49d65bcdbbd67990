"""GPU parity gate for every kernel, through the C ABI (ctypes op module), against the CPU oracle on identical seeded
inputs. Mirrors the reference's tests/test_kernels.py order and tolerances:
  1. 4-row GEMV, closed-form answer, every stage/config, exact                       (test_kernels.py:47-57)
  2. one-hot x sweep over all 128 columns, exact                                    (test_kernels.py:58-68)
  3. real GEMV shapes x group sizes vs fp32 matvec of the dequantized weight, 5e-3  (test_kernels.py:71-86)
  4. paged attention at ctx 128 / odd contexts / 512..16K flat+peaky / spare splits, 2e-3  (test_kernels.py:89-147)
  5. fused norm / swiglu / rope+append (residual and v-copy exact)                   (test_kernels.py:150-176)
plus what the reference does not test: the GPU quantizer bit-exact against the oracle, head_dim 128, the argmax step
kernel and graph replay of the ops. Error metric: normwise max_rel = max|out - ref| / max|ref|.
"""
import zlib

import numpy as np
import pytest
import torch

from helpers import DEV, assert_close, dequant_from_gpu, err, gen, make_cache
from oracle import quant_ref as Q
from oracle import ref_ops as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


# (stage, R, warps, pf): the exact-dequant rung, the R=1 rung, the whole-row streaming kernel over rows x waves x
# prefetch depth, and the split-K kernel over rows x waves x prefetch
GEMV_CFGS = [(0, 1, 4, 0), (0, 1, 1, 0), (1, 1, 0, 0), (1, 1, 4, 3)] + \
            [(2, r, w, pf) for r in (1, 2, 4, 8) for w in (1, 4) for pf in (0, 1, 2, 3)] + \
            [(3, r, w, pf) for r in (1, 2, 4, 8) for w in (0, 1, 4) for pf in (0, 1)] + \
            [(4, r, 0, pf) for r in (1, 2, 4, 8) for pf in (0, 1, 2, 3)] + [(4, 4, 16, 1)]


def tile_groups(Kd, cfgs=((4, 1, 2, 1), (4, 2, 4, 1), (4, 4, 2, 2), (4, 2, 16, 0))):
    """Stage-4 configurations with several row groups per workgroup, their `warps` scaled to whole row groups of
    ceil(Kd / 2048) waves (those that fit 16 waves); the rest of a list passes through."""
    tw = -(-Kd // 2048)
    out = []
    for c in cfgs:
        if c[0] != 4 or c[2] == 0:
            out.append(c)
        elif c[2] * tw <= 16:
            out.append((4, c[1], c[2] * tw, c[3]))
    return out


def gemv(K, cfg, packed, sz, x, N, group):
    y = torch.empty(N, dtype=torch.half, device=DEV)
    K.gemv_w4a16(cfg[0], cfg[1], cfg[2], cfg[3], packed, sz, x, y, group)
    return y


def _shape1():
    N, Kd = 4, 128
    q = np.array([[(k + r) % 16 for k in range(Kd)] for r in range(N)], np.uint8)
    s = np.array([[(r + 1) * 0.5] for r in range(N)], np.float16)
    z = np.full((N, 1), 8.0, np.float16)
    return q, s, z


@pytest.mark.parametrize("cfg", GEMV_CFGS)
def test_gemv_shape1_and_onehot(K, cfg):
    q, s, z = _shape1()
    packed = torch.from_numpy(Q.pack(q)).to(DEV)
    sz = torch.from_numpy(Q.pack_scale_zero(s, z)).to(DEV)
    y = gemv(K, cfg, packed, sz, torch.ones(128, dtype=torch.half, device=DEV), 4, 128)
    assert y.float().cpu().tolist() == [-32.0, -64.0, -96.0, -128.0], cfg
    xs = torch.eye(128, dtype=torch.half, device=DEV)
    ys = torch.stack([gemv(K, cfg, packed, sz, xs[k].contiguous(), 4, 128) for k in range(128)])  # [k, r]
    want = (torch.from_numpy(q.astype(np.float32)).t() - 8) * torch.from_numpy(s[:, 0].astype(np.float32))
    bad = int((ys.float().cpu() != want).any(dim=1).sum())
    assert bad == 0, f"{cfg}: {bad} wrong columns"


SHAPES = {"qkv": (2560, 2048), "o": (2048, 2048), "gate_up": (11264, 2048), "down": (2048, 5632),
          "lm_head": (32000, 2048), "cfg1": (5632, 2048)}       # cfg1: BASELINE config 1, the plain 5632 x 2048 GEMV
SHAPES_8B = {"qkv8b": (6144, 4096), "o8b": (4096, 4096), "down8b": (4096, 14336), "up8b": (14336, 4096)}
# one GPU's share of each projection under tensor parallelism (Llama-3-8B over 8 GPUs, TinyLlama over 4)
SHAPES_TP = {"qkv8b_tp8": (768, 4096), "o8b_tp8": (4096, 512), "gate_up8b_tp8": (3584, 4096),
             "down8b_tp8": (4096, 1792), "qkv_tp4": (640, 2048), "o_tp4": (2048, 512), "gate_up_tp4": (2816, 2048),
             "down_tp4": (2048, 1408)}


def _quantized(K, N, Kd, G, seed):
    w = (torch.randn(N, Kd, generator=gen(seed)) * 0.02).half()
    packed = torch.empty(N, Kd // 8, dtype=torch.int32, device=DEV)
    sz = torch.empty(N, Kd // G, 2, dtype=torch.half, device=DEV)
    K.quantize_w4(w.to(DEV), packed, sz, G)
    return w, packed, sz


# the TinyLlama shapes at three group sizes, the Llama-3-8B shapes and the tensor-parallel shard shapes at the
# models' group size
@pytest.mark.parametrize("name,G", [(n, g) for g in (64, 128, 256) for n in SHAPES] + [(n, 128) for n in SHAPES_8B]
                         + [(n, 128) for n in SHAPES_TP])
def test_gemv_real_shapes(K, name, G):
    N, Kd = {**SHAPES, **SHAPES_8B, **SHAPES_TP}[name]
    w, packed, sz = _quantized(K, N, Kd, G, seed=zlib.crc32(name.encode()) % 1000)
    wref = dequant_from_gpu(packed, sz, G)
    x = torch.randn(Kd, generator=gen(1)).half()
    ref = R.gemv_ref(wref, x)
    xd = x.to(DEV)
    cfgs = GEMV_CFGS if (G == 128 and name in SHAPES) else [(0, 1, 4, 0), (1, 1, 0, 0), (2, 4, 0, 0), (2, 8, 2, 1),
                                                           (2, 2, 1, 3), (3, 4, 0, 0), (3, 2, 1, 1), (4, 2, 0, 0),
                                                           (4, 8, 0, 3)]
    from runtime.model import default_gemv_config
    cfgs = [c for c in cfgs if not (c[0] == 4 and c[2])] + tile_groups(Kd) + [default_gemv_config(N, Kd)]
    for cfg in cfgs:
        assert_close(gemv(K, cfg, packed, sz, xd, N, G), ref, 5e-3, f"gemv {name} {N}x{Kd} G{G} {cfg}")


@pytest.mark.parametrize("N,Kd,G", [(64, 256, 32), (96, 1024, 64), (5632, 2048, 128), (2560, 2048, 256),
                                    (33, 4096, 512), (4096, 14336, 128)])
def test_quantize_bit_exact(K, N, Kd, G):
    """GPU RTN quantize + pack == oracle quantize + pack, bit for bit (codes, scale, zero)."""
    g = gen(N * 7 + Kd)
    w = (torch.randn(N, Kd, generator=g) * 0.02).half()
    w[0, :G] = 0.0                      # all-zero group: scale floor
    if Kd >= 2 * G:
        w[1 % N, G:2 * G] = 0.7         # constant group: zero clamps
    packed = torch.empty(N, Kd // 8, dtype=torch.int32, device=DEV)
    sz = torch.empty(N, Kd // G, 2, dtype=torch.half, device=DEV)
    K.quantize_w4(w.to(DEV), packed, sz, G)
    rows = np.arange(N) if N * Kd <= 16 << 20 else np.random.default_rng(0).choice(N, 256, replace=False)
    wn = w.numpy()[rows]
    q, s, z = Q.quantize(wn, G)
    assert np.array_equal(packed.cpu().numpy()[rows], Q.pack(q))
    assert np.array_equal(sz.cpu().numpy()[rows].view(np.uint16), Q.pack_scale_zero(s, z).view(np.uint16))


def test_quantize_ties(K):
    """Round-half-even ties (scale 0.5, w/scale in {0.5, 1.5, 2.5}; zero-point tie) reproduce the oracle's codes."""
    w = torch.tensor([[-0.5, 7.0, 0.25, 0.75, 1.25, 0.0, 0.0, 0.0] * 4,
                      [-0.25, 7.25, 0, 0, 0, 0, 0, 0] * 4], dtype=torch.half)
    packed = torch.empty(2, 4, dtype=torch.int32, device=DEV)
    sz = torch.empty(2, 1, 2, dtype=torch.half, device=DEV)
    K.quantize_w4(w.to(DEV), packed, sz, 32)
    q, s, z = Q.quantize(w.numpy(), 32)
    assert np.array_equal(packed.cpu().numpy(), Q.pack(q))
    assert Q.unpack(packed.cpu().numpy())[0, :8].tolist() == [0, 15, 1, 3, 3, 1, 1, 1]
    assert sz.cpu().float().tolist() == [[[0.5, 1.0]], [[0.5, 0.0]]]


# ---------------------------------------------------------------------------------------------------- attention
def close_or_rejected(out, ref, tol, what):
    if out is not None:
        assert_close(out, ref, tol, what)


def lean_fits(PS, page, D):
    """version 5 / impl 3: pages of >= 16 tokens, part sizes a multiple of 16 up to 512 (256 at head_dim 128)."""
    return page >= 16 and PS % 16 == 0 and PS <= (256 if D == 128 else 512)


def run_attn(K, q, kc, vc, bt, ctx, PS, version=3, spare=0):
    """spare > 0 sizes the split buffers for more splits than ctx needs, as the runtime does. A part size the lean
    MFMA kernel (version 5) cannot take must be rejected: then the call is checked to raise and None is returned."""
    if version == 5 and not lean_fits(PS, kc.shape[2], kc.shape[3]):
        with pytest.raises(RuntimeError, match="version 5 needs pages"):
            _run_attn(K, q, kc, vc, bt, ctx, PS, version, spare)
        return None
    return _run_attn(K, q, kc, vc, bt, ctx, PS, version, spare)


def _run_attn(K, q, kc, vc, bt, ctx, PS, version, spare):
    D = kc.shape[-1]
    n_q = q.numel() // D
    max_splits = max(1, (ctx + PS - 1) // PS) + spare
    o_part = torch.empty(n_q, max_splits, D, device=DEV)
    m_part = torch.empty(n_q, max_splits, device=DEV)
    l_part = torch.empty_like(m_part)
    out = torch.empty(n_q, D, dtype=torch.half, device=DEV)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=DEV)
    K.paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), pos, PS, o_part, m_part, l_part, out, version)
    return out


@pytest.mark.parametrize("n_q,n_kv", [(32, 4), (8, 8), (16, 4), (8, 4)])
@pytest.mark.parametrize("page", (16, 32))
def test_attention_ctx128(K, n_q, n_kv, page):
    kc, vc, bt = make_cache(128, n_kv, page, seed=n_q + page)
    q = torch.randn(n_q, 64, generator=gen(5)).half()
    k, v = R.gather_kv(kc, vc, bt, 128, page)
    ref = R.attention_contiguous_ref(q, k, v)
    for PS in (4096, 64, 32, 48, 16):
        for ver in (1, 2, 3, 4, 5):
            close_or_rejected(run_attn(K, q, kc, vc, bt, 128, PS, ver), ref, 2e-3,
                         f"ctx128 {n_q}/{n_kv} P{page} PS{PS} v{ver}")


@pytest.mark.parametrize("ctx", (1, 2, 17, 63, 65, 129, 1000))
@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_odd_ctx(K, ver, ctx):
    kc, vc, bt = make_cache(ctx, 4, 16, seed=ctx)
    q = torch.randn(32, 64, generator=gen(ctx + 1)).half()
    ref = R.paged_attention_ref(q, kc, vc, bt, ctx, 16)
    for PS in (8192, 64, 256):
        close_or_rejected(run_attn(K, q, kc, vc, bt, ctx, PS, ver), ref, 2e-3, f"ctx{ctx} PS{PS} v{ver}")


@pytest.mark.parametrize("ctx", (512, 1024, 2048, 4096, 8192, 16384))
@pytest.mark.parametrize("peaky", (1.0, 6.0))
@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_real_ctx(K, ver, ctx, peaky):
    kc, vc, bt = make_cache(ctx, 4, 16, peaky=peaky, seed=ctx)
    q = torch.randn(32, 64, generator=gen(ctx + 2)).half()
    ref = R.paged_attention_ref(q, kc, vc, bt, ctx, 16)
    for PS in sorted({ctx, 1024, 256, 128, 64, 32}):
        close_or_rejected(run_attn(K, q, kc, vc, bt, ctx, PS, ver), ref, 2e-3, f"ctx{ctx} peaky{peaky} PS{PS} v{ver}")


@pytest.mark.parametrize("ctx", (1, 40, 64, 100, 700, 2048, 5000))
@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_runtime_spare_splits(K, ver, ctx):
    kc, vc, bt = make_cache(ctx, 4, 16, peaky=6.0, seed=ctx + 3)
    q = torch.randn(32, 64, generator=gen(ctx + 4)).half()
    ref = R.paged_attention_ref(q, kc, vc, bt, ctx, 16)
    for PS in (32, 64, 128, 256):
        close_or_rejected(run_attn(K, q, kc, vc, bt, ctx, PS, ver, spare=8), ref, 2e-3, f"runtime ctx{ctx} PS{PS} v{ver}")


@pytest.mark.parametrize("n_q,n_kv", [(32, 8), (8, 8), (16, 8), (64, 8)])
@pytest.mark.parametrize("ctx", (1, 100, 777, 4096))
@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_head_dim_128(K, ver, n_q, n_kv, ctx):
    kc, vc, bt = make_cache(ctx, n_kv, 16, D=128, peaky=2.0, seed=ctx + n_q)
    q = torch.randn(n_q, 128, generator=gen(ctx)).half()
    ref = R.paged_attention_ref(q, kc, vc, bt, ctx, 16)
    for PS in (ctx, 64, 256):
        close_or_rejected(run_attn(K, q, kc, vc, bt, ctx, PS, ver), ref, 2e-3, f"D128 {n_q}/{n_kv} ctx{ctx} PS{PS} v{ver}")


# every multiple-of-16 band the lean kernel takes at each head dim (the attention policy picks among them): 1-8 waves
# of 1, 2 or 4 tiles with idle tile slots (e.g. 80 = 5 tiles on 8 waves, 160 = 10 tiles on 8 waves x 2, 320 = 20 on
# 8 x 4), with spare splits
@pytest.mark.parametrize("D,n_q,n_kv", [(64, 32, 4), (128, 32, 8)])
@pytest.mark.parametrize("ctx", (700, 2100))
def test_attention_lean_part_bands(K, D, n_q, n_kv, ctx):
    kc, vc, bt = make_cache(ctx, n_kv, 16, D=D, peaky=3.0, seed=ctx + D)
    q = torch.randn(n_q, D, generator=gen(ctx + D)).half()
    ref = R.paged_attention_ref(q, kc, vc, bt, ctx, 16)
    for PS in (48, 80, 96, 112, 144, 160, 176, 192, 208, 224, 240) + ((320, 384, 448) if D == 64 else ()):
        close_or_rejected(run_attn(K, q, kc, vc, bt, ctx, PS, 5, spare=2), ref, 2e-3, f"D{D} ctx{ctx} PS{PS} lean")


@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_ctx1_is_v0(K, ver):
    """Softmax over one token returns that token's V exactly (fp16 in, fp16 out)."""
    kc, vc, bt = make_cache(1, 4, 16, seed=9)
    q = torch.randn(32, 64, generator=gen(9)).half()
    out = run_attn(K, q, kc, vc, bt, 1, 64, ver).cpu()
    v0 = vc[bt[0], :, 0]                          # [n_kv, D]
    assert torch.equal(out, v0.repeat_interleave(8, dim=0))


@pytest.mark.parametrize("ver", (3, 4, 5))
def test_attention_split_buffers_ignored_past_live(K, ver):
    """Splits beyond ceil(ctx/PS) must not touch the buffers (grid sized for the cap, surplus splits exit)."""
    ctx, PS, spare = 100, 32, 6
    kc, vc, bt = make_cache(ctx, 4, 16, seed=11)
    q = torch.randn(32, 64, generator=gen(11)).half()
    ms = (ctx + PS - 1) // PS + spare
    o_part = torch.full((32, ms, 64), 7.0, device=DEV)
    m_part = torch.full((32, ms), 7.0, device=DEV)
    l_part = torch.full((32, ms), 7.0, device=DEV)
    out = torch.empty(32, 64, dtype=torch.half, device=DEV)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=DEV)
    K.paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), pos, PS, o_part, m_part, l_part, out, ver)
    live = (ctx + PS - 1) // PS
    assert torch.all(o_part[:, live:] == 7.0) and torch.all(m_part[:, live:] == 7.0)
    assert_close(out, R.paged_attention_ref(q, kc, vc, bt, ctx, 16), 2e-3, "spare")


# ----------------------------------------------------------------------------------------------- fused elementwise
# 1, 2, 4 and 8 chunks per thread, partial last chunk rounds (8200, 32776) and the largest row (65536)
@pytest.mark.parametrize("H", (2048, 4096, 64, 8200, 16384, 32776, 65536, 65544, 200008))  # > 65536: two-pass kernel
def test_add_rmsnorm(K, H):
    g = gen(H)
    w = (1 + 0.1 * torch.randn(H, generator=g)).half()
    x = (torch.randn(H, generator=g) * 3).half()
    d = torch.randn(H, generator=g).half()
    xr, outr = R.add_rmsnorm_ref(x.clone(), d, w, 1e-5)
    xk, out = x.to(DEV), torch.empty(H, dtype=torch.half, device=DEV)
    K.add_rmsnorm(xk, d.to(DEV), w.to(DEV), out, 1e-5)
    assert torch.equal(xk.cpu(), xr), "residual must be bit-exact"
    assert_close(out, outr, 2e-3, "add_rmsnorm out")
    xk = x.to(DEV)
    K.add_rmsnorm(xk, None, w.to(DEV), out, 1e-5)
    assert torch.equal(xk.cpu(), x), "no-residual norm must not modify x"
    assert_close(out, R.add_rmsnorm_ref(x, None, w, 1e-5)[1], 2e-3, "rmsnorm (no residual)")


@pytest.mark.parametrize("I", (5632, 14336, 8))
def test_swiglu(K, I):
    gu = (torch.randn(2 * I, generator=gen(I)) * 2).half()
    out = torch.empty(I, dtype=torch.half, device=DEV)
    K.swiglu(gu.to(DEV), out)
    assert_close(out, R.swiglu_ref(gu), 2e-3, "swiglu")


@pytest.mark.parametrize("D,n_q,n_kv,theta", [(64, 32, 4, 1e4), (128, 32, 8, 5e5)])
@pytest.mark.parametrize("pos", (0, 1, 37, 2047, 4095))
def test_rope_append(K, D, n_q, n_kv, theta, pos):
    """q and k are bit-exact (fp32 products rounded separately, as the reference's elementwise ops); v copy exact."""
    page = 16
    cos, sin = R.rope_tables(4096, D, theta)
    kc, vc, bt = make_cache(4096, n_kv, page, D=D, seed=pos)
    kr_c, vr_c = kc.clone(), vc.clone()
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(pos + D)).half()
    qref = R.rope_append_ref(qkv.clone(), cos, sin, pos, kr_c, vr_c, bt, n_q, n_kv, D, page)
    qk, kcd, vcd = qkv.to(DEV), kc.to(DEV), vc.to(DEV)
    K.rope_append(qk, cos.to(DEV), sin.to(DEV), torch.tensor([pos], dtype=torch.int32, device=DEV), bt.to(DEV),
                  kcd, vcd, n_q, n_kv)
    assert torch.equal(qk[: n_q * D].view(n_q, D).cpu(), qref), f"rope q pos{pos}: {err(qk[:n_q * D].view(n_q, D), qref)}"
    assert torch.equal(kcd.cpu(), kr_c), f"rope k-cache pos{pos}: {err(kcd, kr_c)}"
    assert torch.equal(vcd.cpu(), vr_c), f"rope v-cache pos{pos}"
    assert torch.equal(qk[n_q * D:].cpu(), qkv[n_q * D:]), "k and v slots of qkv must be untouched"


def test_rope_out_of_table_position_is_noop(K):
    """*pos beyond the rope table: nothing is touched (no out-of-bounds table read)."""
    cos, sin = R.rope_tables(64, 64)
    kc, vc, bt = make_cache(64, 4, 16, seed=3)
    qkv = torch.randn(40 * 64, generator=gen(3)).half()
    qk, kcd = qkv.to(DEV), kc.to(DEV)
    K.rope_append(qk, cos.to(DEV), sin.to(DEV), torch.tensor([64], dtype=torch.int32, device=DEV), bt.to(DEV),
                  kcd, vc.to(DEV), 32, 4)
    assert torch.equal(qk.cpu(), qkv) and torch.equal(kcd.cpu(), kc)


@pytest.mark.parametrize("V", (32000, 128256, 7))
def test_argmax_advance(K, V):
    logits = torch.randn(V, generator=gen(V)).half()
    logits[V // 3] = 50.0
    logits[V // 2] = 50.0                      # tie: the lower index wins, as torch.argmax on the CPU
    tok = torch.zeros(1, dtype=torch.long, device=DEV)
    pos = torch.tensor([41], dtype=torch.int32, device=DEV)
    K.argmax_advance(logits.to(DEV), tok, pos)
    assert int(tok) == int(torch.argmax(logits.float())) == V // 3 and int(pos) == 42
    K.argmax_advance(logits.to(DEV), tok, None)
    assert int(pos) == 42


@pytest.mark.parametrize("V", (1, 5, 8, 9, 31999, 32000, 128256))
@pytest.mark.parametrize("offset", (0, 1, 3, 7))
def test_argmax_edges(K, V, offset):
    """Unaligned starts (scalar head), V % 8 tails, maxima in the head / tail / across batches, NaN (ranks highest,
    first NaN wins) and an all -inf vector (index 0), each against torch.argmax on the CPU."""
    base = torch.randn(V + offset, generator=gen(V * 8 + offset)).half()
    cases = [base.clone()]
    for where in (0, V - 1, V // 2, min(V - 1, 9000)):
        t = base.clone()
        t[offset + where] = 60.0
        cases.append(t)
    t = base.clone()
    t[offset + V - 1] = float("nan")
    t[offset + V // 3] = float("nan")
    cases.append(t)
    cases.append(torch.full((V + offset,), float("-inf"), dtype=torch.half))
    tok = torch.zeros(1, dtype=torch.long, device=DEV)
    for c in cases:
        dev = c.to(DEV)[offset:]
        K.argmax_advance(dev, tok, None)
        assert int(tok) == int(torch.argmax(c[offset:].float())), (V, offset)


@pytest.mark.parametrize("V", (1, 5, 9, 4095, 4096, 4097, 31999, 32000, 128256))
@pytest.mark.parametrize("offset", (0, 3))
def test_argmax_split(K, V, offset):
    """The multi-workgroup pick against torch.argmax on the CPU and against the one-workgroup kernel: the cases of
    test_argmax_edges plus maxima on workgroup borders (4096 logits each) and exact ties across workgroups; the work
    buffer is zero again after every call, so back-to-back calls (and graph replays) start clean."""
    base = torch.randn(V + offset, generator=gen(V * 16 + offset)).half()
    cases = [base.clone()]
    for where in (0, V - 1, V // 2, min(V - 1, 4095), min(V - 1, 4096)):
        t = base.clone()
        t[offset + where] = 60.0
        cases.append(t)
    t = base.clone()
    for where in (V - 1, V // 3, min(V - 1, 4100)):
        t[offset + where] = 61.0                    # ties across workgroups: the lowest index wins
    cases.append(t)
    t = base.clone()
    t[offset + V - 1] = float("nan")
    t[offset + V // 3] = float("nan")
    cases.append(t)
    t = torch.full((V + offset,), -0.0, dtype=torch.half)
    t[offset + V - 1] = 0.0                         # -0 and +0 compare equal: index 0 wins
    cases.append(t)
    cases.append(torch.full((V + offset,), float("-inf"), dtype=torch.half))
    tok, tok1 = (torch.zeros(1, dtype=torch.long, device=DEV) for _ in range(2))
    pos = torch.tensor([7], dtype=torch.int32, device=DEV)
    work = torch.zeros(2, dtype=torch.long, device=DEV)
    for i, c in enumerate(cases):
        dev = c.to(DEV)[offset:]
        K.argmax_advance_split(dev, tok, pos, work)
        K.argmax_advance(dev, tok1, None)
        want = int(torch.argmax(c[offset:].float()))
        assert int(tok) == want == int(tok1), (V, offset, i)
        assert int(pos) == 8 + i and not work.any()


def test_argmax_split_in_graph(K):
    """Captured once, replayed with new logits between replays: every replay picks anew (the work buffer resets)."""
    V = 128256
    logits = torch.randn(V, device=DEV).half()
    tok = torch.zeros(1, dtype=torch.long, device=DEV)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    work = torch.zeros(2, dtype=torch.long, device=DEV)
    K.argmax_advance_split(logits, tok, pos, work)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.argmax_advance_split(logits, tok, pos, work)
    for r in range(5):
        logits.copy_(torch.randn(V, generator=gen(r)).half().to(DEV))
        g.replay()
        torch.cuda.synchronize()
        assert int(tok) == int(torch.argmax(logits.float().cpu())) and int(pos) == 2 + r and not work.any()


def test_graph_replay_of_ops(K):
    """rope -> attention -> GEMV captured into one hipGraph; each replay (with eager work between replays) equals the
    eager result, and the graph reads the device-resident position anew on every replay."""
    n_q, n_kv, D, page, ctx_cap, PS = 32, 4, 64, 16, 256, 32
    cos, sin = (t.to(DEV) for t in R.rope_tables(ctx_cap + 1, D))
    kc, vc, bt = (t.to(DEV) for t in make_cache(ctx_cap, n_kv, page, seed=21))
    w, packed, sz = _quantized(K, 512, n_q * D, 128, seed=21)
    qkv0 = torch.randn((n_q + 2 * n_kv) * D, generator=gen(22)).half().to(DEV)
    qkv = qkv0.clone()
    pos = torch.tensor([100], dtype=torch.int32, device=DEV)
    ms = ctx_cap // PS
    o_part = torch.empty(n_q, ms, D, device=DEV)
    m_part = torch.empty(n_q, ms, device=DEV)
    l_part = torch.empty_like(m_part)
    attn = torch.empty(n_q, D, dtype=torch.half, device=DEV)
    y = torch.empty(512, dtype=torch.half, device=DEV)

    def body():
        K.rope_append(qkv, cos, sin, pos, bt, kc, vc, n_q, n_kv)
        K.paged_attention(qkv[: n_q * D], kc, vc, bt, pos, PS, o_part, m_part, l_part, attn, 3)
        K.gemv_w4a16(2, 4, 0, 0, packed, sz, attn.view(-1), y, 128)

    expected = {}
    for p in (100, 101, 150):
        qkv.copy_(qkv0)
        pos.fill_(p)
        body()
        torch.cuda.synchronize()
        expected[p] = y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for rep in range(3):
        for p in (100, 101, 150):
            qkv.copy_(qkv0)
            pos.fill_(p)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, expected[p]), (rep, p)
            _ = (qkv0.float() * 2).sum().item()     # eager work between replays


# --------------------------------------------------------------------------------- fused-prologue GEMVs (stage 4)
@pytest.mark.parametrize("N,Kd", [(2560, 2048), (11264, 2048), (6144, 4096), (1000, 5632), (4096, 14336)])
@pytest.mark.parametrize("mode", ("delta", "no_delta", "row"))
def test_gemv_rmsnorm_fused(K, N, Kd, mode):
    """y = W . add_rmsnorm(x, delta, w) in one launch vs the oracle's add_rmsnorm_ref then gemv_ref; the residual
    written to x_out is bit-exact (fp16 add); the embedding-row gather reads row *tok of a table."""
    G = 128
    w, packed, sz = _quantized(K, N, Kd, G, seed=N % 97 + Kd)
    wref = dequant_from_gpu(packed, sz, G)
    g = gen(N + Kd)
    table = (torch.randn(7, Kd, generator=g) * 2).half()
    x = table[3].clone()
    d = torch.randn(Kd, generator=g).half() if mode == "delta" else None
    nw = (1 + 0.1 * torch.randn(Kd, generator=g)).half()
    xr, normed = R.add_rmsnorm_ref(x, d, nw, 1e-5)
    ref = R.gemv_ref(wref, normed)
    y = torch.empty(N, dtype=torch.half, device=DEV)
    x_out = torch.zeros(Kd, dtype=torch.half, device=DEV)
    for cfg in ((4, 2, 0, 0), (4, 1, 0, 1), (4, 4, 0, 3), (4, 8, 0, 2)) + tuple(tile_groups(Kd)):
        if mode == "row":
            K.gemv_w4a16_rmsnorm(*cfg, packed, sz, table.to(DEV), torch.tensor([3], device=DEV), None, nw.to(DEV),
                                 1e-5, x_out, y, G)
        else:
            K.gemv_w4a16_rmsnorm(*cfg, packed, sz, x.to(DEV), None, None if d is None else d.to(DEV), nw.to(DEV),
                                 1e-5, x_out, y, G)
        assert_close(y, ref, 5e-3, f"gemv_rmsnorm {mode} {N}x{Kd} {cfg}")
        assert torch.equal(x_out.cpu(), xr), f"residual {mode} {cfg}"


@pytest.mark.parametrize("I,Kd", [(5632, 2048), (14336, 4096), (40, 256), (1000, 5632)])
@pytest.mark.parametrize("norm", (False, True))
def test_gemv_gate_up_swiglu_epilogue(K, I, Kd, norm):
    """act = swiglu(W_gu . x) in one launch over interleaved gate/up rows. Against the oracle (gemv_ref then
    swiglu_ref on the [gate; up] stack) within the GEMV tolerance, and bit-exact against the two separate HIP ops
    (gemv_w4a16 / gemv_w4a16_rmsnorm on the stacked rows, then swiglu): the epilogue rounds exactly where they do.
    I = 40 and 1000 leave a partial last tile."""
    from runtime.model import interleave_halves
    G = 128
    w, packed, sz = _quantized(K, 2 * I, Kd, G, seed=I + Kd)
    wref = dequant_from_gpu(packed, sz, G)
    pk_il, sz_il = interleave_halves(packed), interleave_halves(sz)
    g = gen(I * 5 + Kd)
    x = (torch.randn(Kd, generator=g) * (1 if norm else 0.5)).half()
    d = torch.randn(Kd, generator=g).half() if norm else None
    nw = (1 + 0.1 * torch.randn(Kd, generator=g)).half() if norm else None
    if norm:
        xr, xin = R.add_rmsnorm_ref(x, d, nw, 1e-5)
    else:
        xin = x
    ref = R.swiglu_ref(R.gemv_ref(wref, xin))
    act = torch.empty(I, dtype=torch.half, device=DEV)
    gu = torch.empty(2 * I, dtype=torch.half, device=DEV)
    sep = torch.empty(I, dtype=torch.half, device=DEV)
    x_out = torch.zeros(Kd, dtype=torch.half, device=DEV) if norm else None
    xd = x.to(DEV)
    for cfg in ((4, 2, 0, 0), (4, 1, 0, 1), (4, 4, 0, 2), (4, 8, 0, 3)) + tuple(tile_groups(Kd)):
        if norm:
            K.gemv_w4a16_gate_up(*cfg, pk_il, sz_il, xd, None, d.to(DEV), nw.to(DEV), 1e-5, x_out, act, G)
            K.gemv_w4a16_rmsnorm(*cfg, packed, sz, xd, None, d.to(DEV), nw.to(DEV), 1e-5,
                                 torch.empty_like(xd), gu, G)
            assert torch.equal(x_out.cpu(), xr), f"residual {cfg}"
        else:
            K.gemv_w4a16_gate_up(*cfg, pk_il, sz_il, xd, None, None, None, 0.0, None, act, G)
            K.gemv_w4a16(*cfg, packed, sz, xd, gu, G)
        K.swiglu(gu, sep)
        assert_close(act, ref, 5e-3, f"gate_up I{I} K{Kd} norm={norm} {cfg}")
        assert torch.equal(act, sep), f"gate_up vs gemv + swiglu I{I} K{Kd} norm={norm} {cfg}"


# ------------------------------------------------------------------------------------------ fp16-weight GEMV (LM head)
F16_CFGS = [(1, 0, 0), (2, 4, 2), (4, 1, 1), (1, 8, 3), (2, 2, 0), (4, 4, 3)]


@pytest.mark.parametrize("N,Kd", [(32000, 2048), (37, 8), (100, 520), (1000, 4096), (513, 1024), (64, 3000)])
def test_gemv_f16(K, N, Kd):
    """y = W . x for fp16 W against the oracle's fp32 matvec (reference/ref_ops.py:10-12 with W as stored), the
    reference's GEMV tolerance 5e-3 normwise. K = 520 / 3000 leave dead chunks in the last lane pass; N = 37 / 513 a
    partial last tile."""
    g = gen(N + 3 * Kd)
    w = (torch.randn(N, Kd, generator=g) * 0.02).half()
    x = torch.randn(Kd, generator=g).half()
    ref = R.gemv_ref(w, x)
    wd, xd = w.to(DEV), x.to(DEV)
    y = torch.empty(N, dtype=torch.half, device=DEV)
    for cfg in F16_CFGS:
        if cfg[0] * (1 << max(0, (-(-Kd // 512) - 1).bit_length())) > 16:
            continue
        y.fill_(7.0)
        K.gemv_f16(*cfg, wd, xd, y)
        assert_close(y, ref, 5e-3, f"gemv_f16 {N}x{Kd} {cfg}")


def test_gemv_f16_onehot_exact(K):
    """One-hot x picks a column of W exactly (every other product is an exact zero)."""
    N, Kd = 300, 1040
    w = (torch.randn(N, Kd, generator=gen(9)) * 3).half()
    wd = w.to(DEV)
    y = torch.empty(N, dtype=torch.half, device=DEV)
    for k in (0, 1, 7, 8, 511, 512, 1039):
        x = torch.zeros(Kd, dtype=torch.half, device=DEV)
        x[k] = 1.0
        for cfg in ((1, 0, 0), (2, 4, 2), (4, 2, 3)):
            K.gemv_f16(*cfg, wd, x, y)
            assert torch.equal(y.cpu(), w[:, k]), (k, cfg)


@pytest.mark.parametrize("N,Kd", [(32000, 2048), (1000, 4096), (77, 520)])
@pytest.mark.parametrize("with_delta", (True, False))
def test_gemv_f16_rmsnorm(K, N, Kd, with_delta):
    """The final add_rmsnorm fused in front of the fp16 GEMV: y against add_rmsnorm_ref then gemv_ref (5e-3), x_out
    bit-exact (fp16 add)."""
    g = gen(N * 3 + Kd)
    w = (torch.randn(N, Kd, generator=g) * 0.02).half()
    x = (torch.randn(Kd, generator=g) * 2).half()
    d = torch.randn(Kd, generator=g).half() if with_delta else None
    nw = (1 + 0.1 * torch.randn(Kd, generator=g)).half()
    xr, normed = R.add_rmsnorm_ref(x, d, nw, 1e-5)
    ref = R.gemv_ref(w, normed)
    wd = w.to(DEV)
    y = torch.empty(N, dtype=torch.half, device=DEV)
    for cfg in ((2, 4, 2), (1, 8, 0), (1, 1, 3)):
        x_out = torch.zeros(Kd, dtype=torch.half, device=DEV)
        K.gemv_f16_rmsnorm(*cfg, wd, x.to(DEV), None if d is None else d.to(DEV), nw.to(DEV), 1e-5, x_out, y)
        assert_close(y, ref, 5e-3, f"gemv_f16_rmsnorm {N}x{Kd} {cfg}")
        assert torch.equal(x_out.cpu(), xr), cfg
    K.gemv_f16_rmsnorm(2, 4, 2, wd, x.to(DEV), None if d is None else d.to(DEV), nw.to(DEV), 1e-5, None, y)
    assert_close(y, ref, 5e-3, "no x_out")


def test_fused_step_equals_unfused_step(K):
    """The decode step with fused prologues / epilogue and the one with separate norm / SwiGLU kernels give the same
    logits (same rounding points; only the sum-of-squares order may differ)."""
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(512, 3, 8, 2, 1024, 700)
    out = []
    for fused, swiglu in ((False, "kernel"), (True, "kernel"), (True, "epilogue")):
        m = Model(SyntheticLlama(shape, seed=4, device=DEV, std=0.05), shape,
                  DecodeConfig(max_ctx=64, device=DEV, fused_gemv=fused, swiglu=swiglu))
        m.prepare(64)
        m.reset(0)
        out.append(m.teacher_force([1, 5, 99, 400, 12], collect_logits=True).float().cpu())
    for o in out[1:]:
        err = ((o - out[0]).abs().max() / out[0].abs().max()).item()
        assert err <= 5e-3, err
    # the gate|up SwiGLU epilogue rounds exactly where the separate swiglu kernel does
    assert torch.equal(out[1], out[2])


# ------------------------------------------------------------------------------- qkv GEMV with the RoPE + append epilogue
@pytest.mark.parametrize("D,n_q,n_kv,norm", [(64, 4, 2, True), (64, 6, 2, False), (128, 4, 1, True),
                                             (128, 2, 2, False)])
def test_gemv_qkv_rope_epilogue(K, D, n_q, n_kv, norm):
    """qkv = W_qkv . x with RoPE + KV append in one launch over rotation-pair rows: bit-exact against the two
    separate HIP ops (gemv_w4a16 / gemv_w4a16_rmsnorm on the reference's row order, then rope_append, whose own test
    holds it to the oracle) for the qkv vector and both caches; positions on mapped pages, on an unmapped page (no
    append) and outside [0, max_pos) (nothing rotated or appended)."""
    from runtime.model import rope_pair_rows, rope_tables
    G, Kd = 64, (256 if D == 64 else 512)
    N = (n_q + 2 * n_kv) * D
    _, packed, sz = _quantized(K, N, Kd, G, seed=N + Kd)
    pk, szp = rope_pair_rows(packed, D), rope_pair_rows(sz, D)
    cos, sin = (t.to(DEV) for t in rope_tables(64, D, 10000.0))
    bt = torch.tensor([3, 0, -1, 5], dtype=torch.int32, device=DEV)  # positions 32..47 sit on an unmapped page
    g = gen(N + D)
    xd = (torch.randn(Kd, generator=g) * (1 if norm else 0.5)).half().to(DEV)
    dd = torch.randn(Kd, generator=g).half().to(DEV) if norm else None
    nwd = (1 + 0.1 * torch.randn(Kd, generator=g)).half().to(DEV) if norm else None
    for pos_v in (0, 21, 37, 63, 64, -1):
        for cfg in ((4, 2, 0, 0), (4, 1, 0, 1), (4, 4, 0, 2)) + tuple(tile_groups(Kd)):
            print(f"qkv rope D{D} n_q{n_q} n_kv{n_kv} norm={norm} pos {pos_v} cfg {cfg}", flush=True)
            pos = torch.tensor([pos_v], dtype=torch.int32, device=DEV)
            kc_a = torch.randn(6, n_kv, 16, D, generator=g).half().to(DEV)
            vc_a = torch.randn(6, n_kv, 16, D, generator=g).half().to(DEV)
            kc_b, vc_b = kc_a.clone(), vc_a.clone()
            qa = torch.empty(N, dtype=torch.half, device=DEV)
            qb = torch.empty(N, dtype=torch.half, device=DEV)
            if norm:
                xo_a, xo_b = torch.empty_like(xd), torch.empty_like(xd)
                K.gemv_w4a16_qkv_rope(*cfg, pk, szp, xd, None, dd, nwd, 1e-5, xo_a, qa, cos, sin, pos, bt, kc_a,
                                      vc_a, n_q, n_kv, G)
                K.gemv_w4a16_rmsnorm(*cfg, packed, sz, xd, None, dd, nwd, 1e-5, xo_b, qb, G)
                assert torch.equal(xo_a, xo_b)
            else:
                K.gemv_w4a16_qkv_rope(*cfg, pk, szp, xd, None, None, None, 0.0, None, qa, cos, sin, pos, bt, kc_a,
                                      vc_a, n_q, n_kv, G)
                K.gemv_w4a16(*cfg, packed, sz, xd, qb, G)
            K.rope_append(qb, cos, sin, pos, bt, kc_b, vc_b, n_q, n_kv)
            assert torch.equal(qa, qb), f"qkv pos {pos_v} {cfg}"
            assert torch.equal(kc_a, kc_b), f"k cache pos {pos_v} {cfg}"
            assert torch.equal(vc_a, vc_b), f"v cache pos {pos_v} {cfg}"


@pytest.mark.parametrize("shape_t", [(256, 2, 4, 2, 512, 1000), (512, 2, 4, 2, 1024, 1000)])
def test_decode_rope_epilogue_matches_default_step(K, shape_t):
    """The decode step with RoPE + append in the qkv GEMV and attention without RoPE gives the default step's logits
    (attention_decode with RoPE inside) within 5e-3 and the same KV cache bit for bit, over 300 teacher-forced
    tokens (several attention splits); head dims 64 and 128."""
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(*shape_t)
    print(f"rope epilogue decode {shape_t}", flush=True)
    sd = SyntheticLlama(shape, seed=3, device=DEV, std=0.05, norm_std=0.1)
    # the attention combine stays a launch of its own in b (combine_in_o off): its merge into the o projection sums
    # in another order and has its own test (tests/test_attn_in_o_gpu.py)
    a = Model(sd, shape, DecodeConfig(max_ctx=512, device=DEV, rope_epilogue=False))
    b = Model(sd, shape, DecodeConfig(max_ctx=512, device=DEV, rope_epilogue=True, combine_in_o=False))
    assert b.rope_epilogue
    for m in (a, b):
        m.prepare(512)
        m.reset(0)
    toks = torch.randint(0, shape.vocab_size, (300,), generator=torch.Generator().manual_seed(0)).tolist()
    la = a.teacher_force(toks, collect_logits=True)
    lb = b.teacher_force(toks, collect_logits=True)
    for i in (0, 1, 150, 299):
        assert_close(lb[i], la[i], 5e-3, f"logits at position {i}")
    rows = a.bt[: (300 + 15) // 16].long()
    assert torch.equal(b.kv[:, :, rows], a.kv[:, :, rows])
