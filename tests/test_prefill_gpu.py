"""GPU parity of the prefill path (the scope's prefill row; the reference has no prefill kernel and teacher-forces
prompts through its decode step): the W4A16 GEMM against the oracle's fp32 product with the dequantized weight (the
reference's GEMV tolerance), one-hot rows bit-exact (each product is an exact fp16 x fp16 product, every other term
an exact zero), the SwiGLU epilogue bit-exact against the plain GEMM followed by the swiglu kernel."""
import numpy as np
import pytest
import torch

from helpers import DEV, assert_close, dequant_from_gpu, gen, make_cache
from oracle import quant_ref as Q
from oracle import ref_ops as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


def _weights(K, N, Kd, G, seed):
    w = (torch.randn(N, Kd, generator=gen(seed)) * 0.02).half()
    packed = torch.empty(N, Kd // 8, dtype=torch.int32, device=DEV)
    sz = torch.empty(N, Kd // G, 2, dtype=torch.half, device=DEV)
    K.quantize_w4(w.to(DEV), packed, sz, G)
    return packed, sz


# kernel coverage: K % 128 == 0 and G >= 64 -> the register-stationary kernel when a tiling has enough tiles:
# 256 weight rows x 128 tokens (the last four cases: G 64, 128 and 256, ragged M and N, an odd chunk count),
# 128 x 128 ((512, 11264), ragged (300, 20000), (260, 19998) with N % 4 != 0 and 3 chunks), 128 x 64 ((512, 2560),
# ragged (130, 10002), (200, 12302) at G 64); otherwise K % 64 == 0 -> the wide kernel, tiles
# 128 x 128, 128 x 64, 64 x 64 and 1, 2 or 4 K groups by grid size (G 32 keeps (512, 4096, 1024) on 128 x 64 with 2
# groups and (200, 4100, 512) on 64 x 64 with 2); K % 64 == 32 -> the 16x16x16 kernel; N % 4 != 0 -> the element-wise
# epilogue stores
@pytest.mark.parametrize("M,N,Kd,G", [(1, 64, 256, 128), (7, 2560, 2048, 128), (64, 2048, 2048, 64),
                                      (100, 1000, 5632, 128), (512, 11264, 2048, 128), (33, 4096, 4096, 32),
                                      (512, 4096, 1024, 128), (70, 999, 256, 128), (40, 300, 320, 64),
                                      (300, 4100, 448, 64), (512, 8192, 192, 64), (20, 100, 96, 32),
                                      (500, 16400, 192, 64), (256, 65536, 256, 64), (512, 16384, 256, 32),
                                      (400, 8000, 256, 32), (200, 12302, 640, 64), (300, 20000, 256, 64),
                                      (260, 19998, 384, 128), (512, 2560, 2048, 128), (130, 10002, 512, 64),
                                      (512, 4096, 1024, 32), (200, 4100, 512, 32),
                                      (300, 49002, 384, 128), (130, 98304, 512, 256), (512, 28672, 1024, 128)])
def test_gemm_matches_oracle(K, M, N, Kd, G):
    packed, sz = _weights(K, N, Kd, G, seed=M + N)
    wref = dequant_from_gpu(packed, sz, G)
    x = torch.randn(M, Kd, generator=gen(M * 3 + Kd)).half()
    ref = (x.float() @ wref.float().t())
    y = torch.full((M, N), 7.0, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, x.to(DEV), y, G)
    assert_close(y, ref, 5e-3, f"gemm {M}x{N}x{Kd} G{G}")


def _grid_weights(N, Kd, G, seed):
    """Codes and zeros uniform in 0..15 and scales 2^-6 or 2^-5 per group (packed by the oracle): every dequantized
    weight is a multiple of 2^-6, so with small-integer x every product and every partial sum of the GEMM is exact in
    fp32 whatever the summation order, and the result is the exact product rounded once to fp16."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, (N, Kd), dtype=np.uint8)
    zero = rng.integers(0, 16, (N, Kd // G)).astype(np.float16)
    scale = np.where(rng.random((N, Kd // G)) < 0.5, 2.0 ** -6, 2.0 ** -5).astype(np.float16)
    packed = torch.from_numpy(Q.pack(q)).to(DEV)
    sz = torch.from_numpy(Q.pack_scale_zero(scale, zero)).to(DEV)
    return packed, sz, torch.from_numpy(Q.dequantize(q, scale, zero, G))


# one case per kernel and tiling: the K % 64 == 32 kernel; the wide kernel at 64 x 64 with 1, 2 and 4 K groups,
# 128 x 64 with 1 and 2, 128 x 128; the register-stationary tilings 256 x 128, 128 x 128, 128 x 64; split-K over
# 256-row tiles (the 256 x 64 tiling runs split only) and over 128-row tiles
@pytest.mark.parametrize("M,N,Kd,G,ws", [(20, 100, 96, 32, False), (40, 300, 320, 64, False),
                                         (200, 4100, 512, 32, False), (64, 2048, 2048, 64, False),
                                         (400, 8000, 256, 32, False), (512, 4096, 1024, 32, False),
                                         (512, 8192, 192, 64, False), (256, 65536, 256, 64, False),
                                         (300, 20000, 256, 64, False), (200, 12302, 640, 64, False),
                                         (130, 10002, 512, 64, False), (300, 4100, 13952, 64, True),
                                         (512, 2048, 5632, 128, True)])
def test_gemm_exact_on_integer_grid(K, M, N, Kd, G, ws):
    """Bit-exact against the oracle where the arithmetic is exact (see _grid_weights): pins every index and every
    term of the reduction, split-K's partials included, independently of the fp32 summation order."""
    packed, sz, wref = _grid_weights(N, Kd, G, seed=M + N + Kd)
    x = torch.randint(-3, 4, (M, Kd), generator=gen(M + 1)).half()
    want = (x.float() @ wref.float().t()).half()        # exact sums (multiples of 2^-6 below 2^18), one rounding
    y = torch.full((M, N), 7.0, dtype=torch.half, device=DEV)
    need = K.gemm_workspace_bytes(M, N, Kd, G)
    assert (need > 0) == ws
    K.gemm_w4a16(packed, sz, x.to(DEV), y, G,
                 workspace=torch.empty(need, dtype=torch.uint8, device=DEV) if ws else None)
    assert torch.equal(y.cpu(), want)


# split-K (a workspace; K long or no unsplit register-stationary tiling; at least 16 k chunks per split): S = 4 over
# 256-row tiles at Llama-3 down, S = 2 over 128-row tiles at TinyLlama down (44 chunks), S = 4 with uneven chunk
# ranges (109 chunks) and ragged M and N, S = 4 at G 256 with M = 100 (its second token tile shifted inward)
@pytest.mark.parametrize("M,N,Kd,G,S", [(512, 4096, 14336, 128, 4), (512, 2048, 5632, 128, 2),
                                        (300, 4100, 13952, 64, 4), (100, 14000, 8192, 256, 4)])
def test_gemm_splitk_matches_oracle(K, M, N, Kd, G, S):
    assert K.gemm_workspace_bytes(M, N, Kd, G) == S * M * N * 4
    packed, sz = _weights(K, N, Kd, G, seed=M + N + 1)
    wref = dequant_from_gpu(packed, sz, G)
    x = torch.randn(M, Kd, generator=gen(M * 5 + Kd)).half()
    ref = (x.float() @ wref.float().t())
    ws = torch.full((S * M * N * 4 + 64,), 0xFF, dtype=torch.uint8, device=DEV)   # NaN-filled: every slot is written
    y = torch.full((M, N), 7.0, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, x.to(DEV), y, G, workspace=ws)
    assert_close(y, ref, 5e-3, f"split-K gemm {M}x{N}x{Kd} G{G} S{S}")
    y2 = torch.empty_like(y)
    K.gemm_w4a16(packed, sz, x.to(DEV), y2, G, workspace=ws)
    assert torch.equal(y, y2)                           # deterministic: the partials are summed in split order
    y3 = torch.empty_like(y)
    K.gemm_w4a16(packed, sz, x.to(DEV), y3, G)          # without a workspace: the unsplit kernel, same tolerance
    assert_close(y3, ref, 5e-3, "unsplit")


# the split partials read by the next residual + RMSNorm instead of the GEMM's reduce launch: S 2 (TinyLlama down),
# S 4 over 32-row tiles with a ragged M, S 8 (two batches of four splits in the norm's loads)
@pytest.mark.parametrize("M,N,Kd,S", [(512, 2048, 5632, 2), (100, 4096, 14336, 4), (256, 1536, 16384, 8)])
def test_rmsnorm_rows_parts_matches_reduce_then_norm(K, M, N, Kd, S):
    """gemm_w4a16_parts leaves S fp32 partials whose split-order sum, rounded once, is the reduced output, and
    rmsnorm_rows_parts over them gives x and the normed rows bit for bit as gemm_w4a16 (workspace) then rmsnorm_rows;
    also for the last row alone (the partials of a slice of rows, strided)."""
    G = 128
    need = K.gemm_workspace_bytes(M, N, Kd, G)
    assert need == S * M * N * 4
    packed, sz = _weights(K, N, Kd, G, seed=M + S)
    a = torch.randn(M, Kd, generator=gen(S)).half().to(DEV)
    x0 = torch.randn(M, N, generator=gen(S + 1)).half().to(DEV)
    w = (torch.rand(N, generator=gen(S + 2)) + 0.5).half().to(DEV)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    y = torch.empty(M, N, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, a, y, G, workspace=ws)
    x1, o1 = x0.clone(), torch.empty_like(x0)
    K.rmsnorm_rows(x1, None, y, w, x1, o1, 1e-5)
    ws.fill_(255)
    parts = K.gemm_w4a16_parts(packed, sz, a, G, ws)
    assert parts.shape == (S, M, N)
    tot = parts[0].clone()
    for s in range(1, S):
        tot += parts[s]
    assert torch.equal(tot.half(), y)
    x2, o2 = x0.clone(), torch.empty_like(x0)
    K.rmsnorm_rows_parts(x2, parts, w, x2, o2, 1e-5)
    assert torch.equal(x2, x1) and torch.equal(o2, o1)
    x3, o3 = x0[-1:].clone(), torch.empty(1, N, dtype=torch.half, device=DEV)
    K.rmsnorm_rows_parts(x3, parts[:, -1:], w, x3, o3, 1e-5)
    assert torch.equal(x3, x1[-1:]) and torch.equal(o3, o1[-1:])


def test_gemm_short_k_does_not_split(K):
    """Shapes whose splits would hold fewer than 16 k chunks run unsplit even with a workspace (TinyLlama's
    projections): no workspace is asked for, and passing one changes nothing, bit for bit."""
    M, N, Kd, G = 512, 2560, 2048, 128
    assert K.gemm_workspace_bytes(M, N, Kd, G) == 0
    packed, sz = _weights(K, N, Kd, G, seed=5)
    x = torch.randn(M, Kd, generator=gen(6)).half().to(DEV)
    y1, y2 = (torch.empty(M, N, dtype=torch.half, device=DEV) for _ in range(2))
    K.gemm_w4a16(packed, sz, x, y1, G)
    K.gemm_w4a16(packed, sz, x, y2, G, workspace=torch.empty(1 << 20, dtype=torch.uint8, device=DEV))
    assert torch.equal(y1, y2)


def test_gemm_splitk_one_hot_rows_exact(K):
    """One-hot rows through the split-K path: each row's single product lands in one split's partial, the others add
    exact zeros, so row i of Y is column k_i of the dequantized weight bit for bit."""
    M, N, Kd, G = 64, 8192, 8192, 64                 # split 4 ways over 128-row tiles
    assert K.gemm_workspace_bytes(M, N, Kd, G) == 4 * M * N * 4
    packed, sz = _weights(K, N, Kd, G, seed=21)
    wref = dequant_from_gpu(packed, sz, G)
    ks = [0, 1, 127, 128, 511, 512, 1000, 1535, 2047, 2048, 4095, 4096, 6143, 6144, 8191] + [700] * (M - 15)
    x = torch.zeros(M, Kd, dtype=torch.half)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    ws = torch.empty(K.gemm_workspace_bytes(M, N, Kd, G), dtype=torch.uint8, device=DEV)
    y = torch.empty(M, N, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, x.to(DEV), y, G, workspace=ws)
    assert torch.equal(y.cpu(), wref[:, ks].t().contiguous())


@pytest.mark.parametrize("N", [200, 49152])
def test_gemm_one_hot_rows_exact(K, N):
    """Row i of X is one-hot at k_i, so row i of Y is column k_i of the dequantized weight, bit for bit (N 49152 runs
    the register-stationary kernel, whose k order within an MFMA step is permuted)."""
    Kd, G = 512, 64
    packed, sz = _weights(K, N, Kd, G, seed=9)
    wref = dequant_from_gpu(packed, sz, G)
    ks = [0, 1, 7, 8, 31, 32, 127, 128, 300, 511] * 6 + [64, 65, 255, 256]   # 64 rows (the kernel's token tile)
    x = torch.zeros(len(ks), Kd, dtype=torch.half)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y = torch.empty(len(ks), N, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, x.to(DEV), y, G)
    assert torch.equal(y.cpu(), wref[:, ks].t().contiguous())


# register-stationary tilings of the SwiGLU epilogue: 128 x 128 at (512, 8192), 256 x 128 at (260, 14000), 128 x 64
# at (64, 20500) and (64, 10240)
@pytest.mark.parametrize("M,I,Kd", [(16, 5632, 2048), (130, 512, 256), (1, 64, 1024), (9, 513, 320), (33, 70, 96),
                                    (512, 8192, 256), (260, 14000, 640), (64, 20500, 256), (64, 10240, 256)])
def test_gemm_swiglu_epilogue(K, M, I, Kd):
    from runtime.model import interleave_halves
    G = 128 if Kd % 128 == 0 else (64 if Kd % 64 == 0 else 32)
    packed, sz = _weights(K, 2 * I, Kd, G, seed=I + M)
    x = torch.randn(M, Kd, generator=gen(I)).half().to(DEV)
    gu = torch.empty(M, 2 * I, dtype=torch.half, device=DEV)
    K.gemm_w4a16(packed, sz, x, gu, G)
    act = torch.empty(M, I, dtype=torch.half, device=DEV)
    K.gemm_w4a16(interleave_halves(packed), interleave_halves(sz), x, act, G, epilogue=1)
    if I % 8 == 0:                                   # the swiglu kernel's shape rule
        sep = torch.empty(M, I, dtype=torch.half, device=DEV)
        for m in range(M):
            K.swiglu(gu[m], sep[m])
        assert torch.equal(act, sep)
    else:
        assert_close(act, R.swiglu_ref(gu.cpu()), 1e-3, "gemm swiglu vs oracle swiglu of the GEMM output")
    ref = R.swiglu_ref((x.cpu().float() @ dequant_from_gpu(packed, sz, G).float().t()).half())
    assert_close(act, ref, 5e-3, "gemm swiglu vs oracle")


# ---------------------------------------------------------------------------------------------------------------
# batched elementwise kernels: bit-exact against their one-token forms, which the decode tests pin to the oracle

def _pos(p):
    return torch.tensor([p], dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("D,n_q,n_kv,page,start,M,max_pos", [(64, 32, 4, 16, 0, 37, 200), (128, 32, 8, 16, 5, 64, 80),
                                                            (64, 8, 8, 32, 100, 1, 200), (64, 16, 4, 16, 60, 20, 75)])
def test_rope_append_rows_matches_per_token(K, D, n_q, n_kv, page, start, M, max_pos):
    """Row m is token start + m; rows at positions >= max_pos (the last case) touch nothing, as the one-token op."""
    cos, sin = (t.to(DEV) for t in R.rope_tables(max_pos, D))
    n_pages = (start + M + page - 1) // page + 2
    bt = torch.randperm(n_pages, generator=gen(D + M)).int().to(DEV)
    qkv = torch.randn(M, (n_q + 2 * n_kv) * D, generator=gen(M + start)).half()
    shape = (n_pages, n_kv, page, D)
    kc1, vc1, kc2, vc2 = (torch.full(shape, -3.0, dtype=torch.half, device=DEV) for _ in range(4))
    a = qkv.clone().to(DEV)
    K.rope_append_rows(a, cos, sin, _pos(start), bt, kc1, vc1, n_q, n_kv)
    rows = []
    for m in range(M):
        r = qkv[m].clone().to(DEV)
        K.rope_append(r, cos, sin, _pos(start + m), bt, kc2, vc2, n_q, n_kv)
        rows.append(r)
    assert torch.equal(a, torch.stack(rows))
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    kr, vr = kc2.cpu().clone().fill_(-3.0), vc2.cpu().clone().fill_(-3.0)
    for m in range(min(M, max_pos - start)):
        q = R.rope_append_ref(qkv[m], cos.cpu(), sin.cpu(), start + m, kr, vr, bt.cpu(), n_q, n_kv, D, page)
        assert torch.equal(a[m, : n_q * D].cpu().view(n_q, D), q)
    assert torch.equal(kc1.cpu(), kr) and torch.equal(vc1.cpu(), vr)


@pytest.mark.parametrize("M,H,gather,with_delta,inplace", [(9, 2048, True, False, False), (33, 4096, False, True, True),
                                                          (1, 256, False, True, False), (130, 2048, True, True, False),
                                                          (3, 16384, True, True, False), (2, 65536, False, False, True)])
def test_rmsnorm_rows_matches_per_row(K, M, H, gather, with_delta, inplace):
    g = gen(M + H)
    src = torch.randn(M + 50 if gather else M, H, generator=g).half().to(DEV)
    rows = torch.randint(0, src.size(0), (M,), generator=g).to(DEV) if gather else None
    delta = torch.randn(M, H, generator=g).half().to(DEV) if with_delta else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).half().to(DEV)
    x_in = src.clone()
    x_out = x_in if inplace else torch.empty(M, H, dtype=torch.half, device=DEV)
    out = torch.empty(M, H, dtype=torch.half, device=DEV)
    K.rmsnorm_rows(x_in, rows, delta, w, x_out, out, 1e-5)
    for m in range(M):
        x = src[int(rows[m]) if gather else m].clone()
        o = torch.empty(H, dtype=torch.half, device=DEV)
        K.add_rmsnorm(x, None if delta is None else delta[m], w, o, 1e-5)
        assert torch.equal(x_out[m], x) and torch.equal(out[m], o), m
        xr, orf = R.add_rmsnorm_ref(src[int(rows[m]) if gather else m].cpu(), None if delta is None else delta[m].cpu(),
                                    w.cpu(), 1e-5)
        assert torch.equal(x.cpu(), xr)
        assert_close(o, orf, 2e-3, f"rmsnorm row {m}")
    if gather:
        assert torch.equal(x_in, src)                 # the gathered source is read only


def test_rmsnorm_rows_out_of_range_gather_is_nan(K):
    """A gathered index outside the source rows is not read: that row comes out NaN, the others are unaffected."""
    H = 256
    src = torch.randn(10, H, generator=gen(77)).half().to(DEV)
    rows = torch.tensor([3, 10, -1, 9], device=DEV)
    w = torch.ones(H, dtype=torch.half, device=DEV)
    x_out = torch.empty(4, H, dtype=torch.half, device=DEV)
    out = torch.empty(4, H, dtype=torch.half, device=DEV)
    K.rmsnorm_rows(src, rows, None, w, x_out, out, 1e-5)
    assert torch.isnan(x_out[1:3]).all() and torch.isnan(out[1:3]).all()
    for m, r in ((0, 3), (3, 9)):
        x = src[r].clone()
        o = torch.empty(H, dtype=torch.half, device=DEV)
        K.add_rmsnorm(x, None, w, o, 1e-5)
        assert torch.equal(x_out[m], x) and torch.equal(out[m], o)


# ---------------------------------------------------------------------------------------------------------------
# causal prefill attention

def _prefill_attn(K, qkv, start, kd, vd, btd, n_q, n_kv, max_ctx):
    D = kd.shape[-1]
    out = torch.full((qkv.shape[0], n_q * D), 9.0, dtype=torch.half, device=DEV)
    K.attention_prefill(qkv.to(DEV), _pos(start), btd, kd, vd, n_q, n_kv, max_ctx, out)
    return out


@pytest.mark.parametrize("D,n_q,n_kv,page,start,M", [(64, 32, 4, 16, 0, 40), (64, 32, 4, 16, 300, 17),
                                                    (128, 32, 8, 16, 0, 64), (128, 8, 8, 32, 1000, 9),
                                                    (64, 16, 8, 16, 0, 1), (64, 4, 4, 16, 4000, 96),
                                                    (128, 16, 4, 16, 20000, 20), (64, 8, 1, 16, 70, 130),
                                                    (64, 64, 32, 16, 0, 300), (128, 64, 32, 16, 100, 280)])
def test_attention_prefill(K, D, n_q, n_kv, page, start, M):
    """Every row m (position start + m) against the oracle's attention over tokens [0, start + m] (2e-3; the cache
    also holds the later rows' tokens, which must not be attended); HPG 1..8, D 64 and 128, contexts past 16K; grids
    of at most 256 workgroups (two wave groups per workgroup, each taking every other block) and, in the last two
    cases, of more (one group)."""
    ctx_all = start + M
    kc, vc, bt = make_cache(ctx_all, n_kv, page, D=D, seed=D + M + start)
    qkv = torch.randn(M, (n_q + 2 * n_kv) * D, generator=gen(start + M)).half()
    kd, vd, btd = kc.to(DEV), vc.to(DEV), bt.to(DEV)
    out = _prefill_attn(K, qkv, start, kd, vd, btd, n_q, n_kv, ctx_all)
    for m in range(M):
        q = qkv[m, : n_q * D].contiguous().view(n_q, D)
        ref = R.paged_attention_ref(q, kc, vc, bt, start + m + 1, page)
        assert_close(out[m].view(n_q, D), ref, 2e-3, f"row {m} vs oracle")


@pytest.mark.parametrize("D,n_q,n_kv,M,ks", [(64, 32, 4, 77, (1, 30, 64, 76)), (64, 64, 32, 300, (1, 20)),
                                             (128, 64, 32, 300, (1, 20))])
def test_attention_prefill_rows_independent_of_batch(K, D, n_q, n_kv, M, ks):
    """A row's result does not depend on which other rows share its launch: the last rows of a prompt computed alone
    (pos advanced, qkv sliced) are bit-identical to the same rows of the whole prompt. Both launches of a case have
    grids on the same side of 256 workgroups (first case below, the others above), which sets the wave groups per
    workgroup and with them the order in which a row's blocks are summed."""
    page = 16
    kc, vc, bt = make_cache(M, n_kv, page, D=D, seed=11 + D)
    qkv = torch.randn(M, (n_q + 2 * n_kv) * D, generator=gen(12)).half()
    kd, vd, btd = kc.to(DEV), vc.to(DEV), bt.to(DEV)
    full = _prefill_attn(K, qkv, 0, kd, vd, btd, n_q, n_kv, M)
    for k in ks:
        part = _prefill_attn(K, qkv[k:].contiguous(), k, kd, vd, btd, n_q, n_kv, M)
        assert torch.equal(part, full[k:]), k


def test_attention_prefill_max_ctx_caps_the_context(K):
    """Tokens at positions >= max_ctx are not attended: rows past the cap see tokens [0, max_ctx)."""
    D, n_q, n_kv, page, M, cap = 64, 8, 2, 16, 40, 25
    kc, vc, bt = make_cache(M, n_kv, page, D=D, seed=13)
    qkv = torch.randn(M, (n_q + 2 * n_kv) * D, generator=gen(14)).half()
    out = _prefill_attn(K, qkv, 0, kc.to(DEV), vc.to(DEV), bt.to(DEV), n_q, n_kv, cap)
    for m in (0, 24, 25, 39):
        q = qkv[m, : n_q * D].contiguous().view(n_q, D)
        ref = R.paged_attention_ref(q, kc, vc, bt, min(m + 1, cap), page)
        assert_close(out[m].view(n_q, D), ref, 2e-3, f"row {m}")


# ---------------------------------------------------------------------------------------------------------------
# Model.prefill

def _model(D=64, **cfg):
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(256, 2, 4, 2, 512, 1000) if D == 64 else LlamaShape(512, 2, 4, 2, 1024, 1000)
    m = Model(SyntheticLlama(shape, seed=4, device=DEV, std=0.05), shape, DecodeConfig(max_ctx=256, device=DEV, **cfg))
    m.prepare(256)
    return m, shape


def _prompt(n, seed=1):
    return torch.randint(0, 1000, (n,), generator=gen(seed))


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("D", (64, 128))
def test_prefill_matches_oracle_and_teacher_force(K, D):
    from __graft_entry__ import _ref_weights
    from oracle.decode_ref import RefDecoder
    m, shape = _model(D)
    prompt = _prompt(45)
    ref = RefDecoder(_ref_weights(m, shape), shape, max_ctx=256, page=16, block_table=m.bt.cpu())
    for p, t in enumerate(prompt.tolist()):
        lr, tr = ref.step(t, p)
    m.reset(0)
    m.prefill(prompt)
    torch.cuda.synchronize()
    assert int(m.pos) == 45 and m.host_pos == 45
    assert _rel(m.logits, lr) <= 2e-2, _rel(m.logits, lr)
    pre_logits, pre_tok, pre_kv = m.logits.clone(), int(m.tok), m.kv.clone()
    m.kv.zero_()
    m.reset(0)
    tf = m.teacher_force(prompt, collect_logits=True)
    assert _rel(pre_logits, tf[-1]) <= 2e-2
    lf = tf[-1].float()
    assert pre_tok == int(m.tok) or lf.max() - lf[pre_tok] <= 2e-2 * lf.abs().max()
    assert _rel(pre_kv, m.kv) <= 2e-2
    # decoding on from the prefilled state follows the oracle
    m.kv.copy_(pre_kv)
    m.tok.fill_(tr)
    m.reset(45)
    for p, t in enumerate((tr, 17, 3), start=45):
        m.tok.fill_(t)
        m.run_step()
        lr, _ = ref.step(t, p)
        assert _rel(m.logits, lr) <= 2e-2, (p, _rel(m.logits, lr))


def test_prefill_in_chunks_is_bit_exact(K):
    """Attention rows are computed independently of their batch, and for this model's shapes every chunk size takes
    the same GEMM configuration (64 x 64 tiles, four K groups; the configuration, and with it the fp32 summation order,
    is chosen per M x N x K) and the same attention grid class (at most 256 workgroups): a prompt prefilled in three
    chunks leaves the same cache and logits as one pass."""
    m, _ = _model()
    prompt = _prompt(70, seed=2)
    m.reset(0)
    m.prefill(prompt)
    one = (m.kv.clone(), m.logits.clone(), int(m.tok), int(m.pos))
    m.kv.fill_(0.5)
    m.reset(0)
    for a, b in ((0, 31), (31, 32), (32, 70)):
        m.prefill(prompt[a:b])
    n = 70 * 1
    used = torch.zeros_like(m.kv, dtype=torch.bool)
    for t in range(n):
        used[:, :, int(m.bt[t // 16]), :, t % 16, :] = True
    assert torch.equal(m.kv[used], one[0][used])
    assert torch.equal(m.logits, one[1]) and int(m.tok) == one[2] and int(m.pos) == one[3] == 70


def test_prefill_split_reduce_folded_into_norm(K):
    """A 512-token prompt through a TinyLlama-width model, whose down projection splits K: with the split partials
    summed by the next norm (the default) the prefill leaves the same cache, logits and token as with the GEMM's own
    reduce launch."""
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(2048, 2, 32, 4, 5632, 1000)
    m = Model(SyntheticLlama(shape, seed=6, device=DEV, std=0.05), shape, DecodeConfig(max_ctx=600, device=DEV))
    m.prepare(600)
    assert K.gemm_workspace_bytes(512, 2048, 5632, m.cfg.group) > 0   # the path under test is taken
    prompt = _prompt(512, seed=9)
    out = []
    for fold in (True, False):
        m.fold_split_reduce = fold
        m.kv.zero_()
        m.reset(0)
        m.prefill(prompt)
        torch.cuda.synchronize()
        out.append((m.kv.clone(), m.logits.clone(), int(m.tok)))
    assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1]) and out[0][2] == out[1][2]


def test_prefill_gate_up_layouts_agree(K):
    """swiglu='kernel' keeps the [gate; up] rows for decode; prefill then uses an interleaved copy, so both
    configurations run the same GEMM and agree bit for bit."""
    prompt = _prompt(23, seed=3)
    outs = []
    for sw in ("epilogue", "kernel"):
        m, _ = _model(swiglu=sw)
        m.reset(0)
        m.prefill(prompt)
        outs.append((m.logits.clone(), m.kv.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_prefill_fp16_weights(K):
    from __graft_entry__ import _ref_weights
    from oracle.decode_ref import RefDecoder
    m, shape = _model(weights="fp16")
    prompt = _prompt(12, seed=5)
    ref = RefDecoder(_ref_weights(m, shape), shape, max_ctx=256, page=16, block_table=m.bt.cpu())
    for p, t in enumerate(prompt.tolist()):
        lr, _ = ref.step(t, p)
    m.reset(0)
    m.prefill(prompt)
    assert _rel(m.logits, lr) <= 2e-2


@pytest.mark.parametrize("head", ("fp16", "int4"))
def test_model_bytes_match_byte_model(K, head):
    """The built model's byte count (tensor sizes) equals the shape-only byte model that the CPU tests pin to the
    reference's published figures."""
    from runtime.model import byte_model
    m, shape = _model(lm_head=head)
    assert m.bytes_per_token(300) == byte_model(shape, 300, head=head)["total"]


def test_prefill_rejects_bad_prompts(K):
    m, _ = _model()
    m.reset(0)
    with pytest.raises(ValueError, match="token ids"):
        m.prefill(torch.tensor([3, 1000]))
    m.reset(250)
    with pytest.raises(RuntimeError, match="exceeds max_ctx"):
        m.prefill(_prompt(7))
    m.reset(0)
    m.prefill([])
    assert m.host_pos == 0
    with pytest.raises(ValueError, match="token ids"):
        m.teacher_force([5, -2])
