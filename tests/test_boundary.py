"""CPU checks of the drop-in boundary (no GPU, no compute): the C-ABI library loads, exports every entry point that
include/dk_amd.h declares with the signature the ctypes shim binds, and every argument-validation path of the C layer
(kernels/bindings.cpp:18-88 TORCH_CHECKs) returns its error code and message before any HIP call. The torch-facing
shim rejects non-CUDA tensors with the reference's message."""
import re

import pytest
import torch

from runtime import ext


@pytest.fixture(scope="module")
def lib():
    return ext.open_library()


def declared_entry_points():
    txt = re.sub(r"/\*.*?\*/", "", ext.HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(dk_\w+)\s*\(", txt, flags=re.M)


def test_library_exports_every_declared_symbol(lib):
    names = declared_entry_points()
    assert len(names) >= 10 and "dk_gemv_w4a16" in names and "dk_paged_attention" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(ext.SIGNATURES), "ctypes signatures must cover exactly the header's entry points"


def test_header_arities_match_shim(lib):
    txt = re.sub(r"/\*.*?\*/", "", ext.HEADER.read_text(), flags=re.S)
    for name, (argtypes, _) in ext.SIGNATURES.items():
        m = re.search(rf"{name}\s*\(([^)]*)\)", txt)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), name


def test_runtime_is_torch_runtime(lib):
    """The library resolves libamdhip64 to the HIP runtime torch loaded: one runtime per process."""
    v = lib.dk_runtime_version()
    if torch.version.hip:
        major, minor = (int(t) for t in torch.version.hip.split(".")[:2])
        assert v // 10_000_000 == major and (v // 100_000) % 100 == minor, (v, torch.version.hip)


A16 = 0x10000          # a 16-byte aligned fake address: validation fails before it is ever dereferenced
B16 = 0x20000          # a second one


def _err(lib, rc):
    return rc, lib.dk_last_error().decode()


@pytest.mark.parametrize("args,code,msg", [
    ((0, 3, 0, 0, A16, A16, A16, A16, 4, 128, 128), 4, "R must be 1,2,4,8"),
    ((5, 1, 0, 0, A16, A16, A16, A16, 4, 128, 128), 4, "stage"),
    ((4, 16, 0, 0, A16, A16, A16, A16, 4, 128, 128), 4, "R must be 1,2,4,8"),
    ((4, 4, 0, 4, A16, A16, A16, A16, 4, 128, 128), 4, "pf must be 0..3"),
    ((4, 4, 2, 0, A16, A16, A16, A16, 4, 8192, 128), 3, "multiple of ceil(K / 2048) = 4"),
    ((4, 4, 6, 0, A16, A16, A16, A16, 4, 8192, 128), 3, "whole row groups"),
    ((4, 4, 17, 0, A16, A16, A16, A16, 4, 2048, 128), 4, "warps must be 0..16"),
    ((2, 1, 17, 0, A16, A16, A16, A16, 4, 128, 128), 4, "warps"),
    ((2, 1, 0, 4, A16, A16, A16, A16, 4, 128, 128), 4, "pf must be 0..3"),
    ((3, 1, 0, 2, A16, A16, A16, A16, 4, 128, 128), 4, "pf must be 0 or 1"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 4, 32800, 32), 3, "K <= 32768"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 4, 100, 128), 3, "multiple of 32"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 4, 128, 256), 3, "multiple of 32 and of the group size"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 4, 192, 96), 4, "group must be a power of two"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 4, 256, 16), 4, "group must be >= 32"),
    ((2, 1, 0, 0, A16 + 4, A16, A16, A16, 4, 128, 128), 2, "packed must be 16B aligned"),
    ((2, 1, 0, 0, A16, A16, A16 + 8, A16, 4, 128, 128), 2, "x must be 16B aligned"),
    ((2, 1, 0, 0, None, A16, A16, A16, 4, 128, 128), 1, "null"),
    ((2, 1, 0, 0, A16, A16, A16, A16, 0, 128, 128), 3, "positive"),
])
def test_gemv_validation(lib, args, code, msg):
    rc, m = _err(lib, lib.dk_gemv_w4a16(*args, None))
    assert rc == code and msg in m, (rc, m)


def _attn(lib, **kw):
    a = dict(version=2, q=A16, kc=A16, vc=A16, bt=A16, pos=A16, n_q=32, n_kv=4, head_dim=64, page=16, n_pages=8,
             n_bt=8, part_size=64, max_splits=4, o=A16, m=A16, l=A16, out=A16)
    a.update(kw)
    return _err(lib, lib.dk_paged_attention(*a.values(), None))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(n_q=24), 3, "heads-per-group must be 1/2/4/8"),
    (dict(n_q=30), 3, "heads-per-group"),
    (dict(head_dim=96), 3, "head_dim"),
    (dict(page=12), 4, "page size must be a power of two"),
    (dict(part_size=0), 4, "part_size must be > 0"),
    (dict(version=6), 4, "version must be 1..5"),
    (dict(version=0), 4, "version must be 1..5"),
    (dict(version=5, part_size=40), 4, "version 5 needs pages of >= 16 tokens"),
    (dict(version=5, part_size=1024), 4, "version 5 needs pages"),
    (dict(version=5, page=8), 4, "version 5 needs pages"),
    (dict(version=5, head_dim=128, part_size=512), 4, "multiple of 16 up to 256"),
    (dict(max_splits=0), 3, "max_splits"),
    (dict(kc=A16 + 2), 2, "16B aligned"),
    (dict(bt=None), 1, "null"),
    (dict(n_bt=0), 3, "empty"),
])
def test_attention_validation(lib, kw, code, msg):
    rc, m = _attn(lib, **kw)
    assert rc == code and msg in m, (rc, m)
    # the split kernel alone checks exactly what paged_attention checks
    a = dict(version=2, q=A16, kc=A16, vc=A16, bt=A16, pos=A16, n_q=32, n_kv=4, head_dim=64, page=16, n_pages=8,
             n_bt=8, part_size=64, max_splits=4, o=A16, m=A16, l=A16, out=A16)
    a.update(kw)
    rs, ms = _err(lib, lib.dk_paged_attention_split(*a.values(), None))
    assert rs == code and msg in ms, (rs, ms)


def _gemv_attn(lib, **kw):
    a = dict(stage=4, R=1, warps=4, pf=1, packed=A16, sz=A16, o=A16, m=A16, l=A16, attn=A16, pos=A16, n_bt=8, page=16,
             part_size=64, max_splits=5, max_pos=0, n_q=32, head_dim=64, y=B16, N=2048, K=2048, group=128)
    a.update(kw)
    return _err(lib, lib.dk_gemv_w4a16_attn(*a.values(), None))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(stage=2), 4, "stage 4 only"),
    (dict(K=1024), 3, "K must be n_q * head_dim"),
    (dict(head_dim=96, K=3072), 3, "head_dim"),
    (dict(max_splits=17), 3, "max_splits must be 1..16"),
    (dict(max_splits=0), 3, "max_splits must be 1..16"),
    (dict(warps=2), 3, "one thread per 8 values of x"),                  # 128 threads for 256 chunks
    (dict(warps=16), 3, "at most 8 waves"),                                # more than the kernel's 8 waves
    (dict(n_q=64, K=4096, warps=7), 3, "whole row groups"),               # a multiple of ceil(K / 2048) = 2
    (dict(n_q=64, K=4096, warps=4), 3, "one thread per 8 values"),
    (dict(part_size=0), 4, "part_size"),
    (dict(page=12), 4, "power of two"),
    (dict(n_bt=0), 3, "n_bt"),
    (dict(max_pos=-1), 4, "max_pos"),
    (dict(o=None), 1, "null"),
    (dict(attn=A16 + 8), 2, "16B aligned"),
    (dict(m=A16 + 2), 2, "4B aligned"),
    (dict(l=A16 + 1), 2, "4B aligned"),
    (dict(y=A16), 4, "must not alias"),                                    # y == attn (and the partials)
    (dict(y=B16, o=B16, attn=A16 + 4096), 4, "must not alias"),          # y == o_part
    (dict(y=B16, m=B16, attn=A16 + 4096), 4, "must not alias"),          # y == m_part
])
def test_gemv_attn_validation(lib, kw, code, msg):
    rc, m = _gemv_attn(lib, **kw)
    assert rc == code and msg in m, (rc, m)


def _dec(lib, **kw):
    a = dict(qkv=A16, c=A16, s=A16, max_pos=100, pos=A16, bt=A16, n_bt=8, kc=A16, vc=A16, n_pages=8, page=16, n_q=32,
             n_kv=4, D=64, part_size=64, max_splits=4, impl=0, o=A16, m=A16, l=A16, out=A16)
    a.update(kw)
    return _err(lib, lib.dk_attention_decode(*a.values(), None))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(n_q=24), 3, "heads-per-group must be 1/2/4/8"),
    (dict(D=96), 3, "head_dim"),
    (dict(page=12), 4, "page size must be a power of two"),
    (dict(part_size=0), 4, "part_size must be > 0"),
    (dict(max_splits=0), 3, "max_splits"),
    (dict(impl=4), 4, "impl must be 0, 1 or 3"),
    (dict(impl=3, part_size=40), 4, "impl 3 needs pages of >= 16 tokens"),
    (dict(impl=3, page=8), 4, "impl 3 needs pages"),
    (dict(impl=3, D=128, part_size=512), 4, "multiple of 16 up to 256"),
    (dict(impl=2), 4, "impl must be 0, 1 or 3"),
    (dict(max_pos=0), 3, "empty"),
    (dict(c=None), 1, "null"),
    (dict(qkv=A16 + 2), 2, "16B aligned"),
])
def test_attention_decode_validation(lib, kw, code, msg):
    rc, m = _dec(lib, **kw)
    assert rc == code and msg in m, (rc, m)




def _fused(lib, fn, **kw):
    a = dict(stage=4, R=2, warps=0, pf=0, packed=A16, sz=A16, x=A16, row=None, delta=None, norm_w=A16, eps=1e-5,
             x_out=None, y=B16, N=64, K=256, group=128)
    a.update(kw)
    return _err(lib, fn(*a.values(), None))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(stage=2), 4, "stage 4 only"),
    (dict(N=63), 3, "must be even"),
    (dict(R=1, pf=0), 4, "gate/up pair"),
    (dict(norm_w=None, delta=A16), 4, "belong to the RMSNorm input"),
    (dict(norm_w=None, x_out=B16 + 0x1000), 4, "belong to the RMSNorm input"),
    (dict(x_out=A16), 4, "x_out must not alias"),
    (dict(y=A16), 4, "act must not alias"),
    (dict(norm_w=A16 + 8), 2, "16B aligned"),
    (dict(row=A16 + 4), 2, "row must be 8B aligned"),
    (dict(K=32800, group=32), 3, "K <= 32768"),
    (dict(y=None), 1, "null"),
])
def test_gate_up_validation(lib, kw, code, msg):
    rc, m = _fused(lib, lib.dk_gemv_w4a16_gate_up, **kw)
    assert rc == code and msg in m, (rc, m)


def _qkv_rope(lib, **kw):
    a = dict(stage=4, R=2, warps=0, pf=0, packed=A16, sz=A16, x=A16, row=None, delta=None, norm_w=A16, eps=1e-5,
             x_out=None, qkv=B16, cos_t=A16, sin_t=A16, pos=A16, bt=A16, kc=A16, vc=A16, n_q=4, n_kv=2,
             head_dim=64, page=16, max_pos=64, n_pages=4, n_bt=4, K=256, group=128)
    a.update(kw)
    return _err(lib, lib.dk_gemv_w4a16_qkv_rope(*a.values(), None))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(head_dim=96), 3, "head_dim must be 64 or 128"),
    (dict(n_kv=0), 3, "bad head counts"),
    (dict(stage=3), 4, "stage 4 only"),
    (dict(R=1, pf=0), 4, "rotation pair"),
    (dict(cos_t=None), 1, "null pointer"),
    (dict(vc=None), 1, "null pointer"),
    (dict(page=24), 4, "power of two"),
    (dict(max_pos=0), 3, "empty rope table"),
    (dict(n_bt=0), 3, "empty rope table"),
    (dict(norm_w=None, delta=A16), 4, "RMSNorm input"),
    (dict(x=A16 + 2), 2, "16B aligned"),
    (dict(qkv=A16), 4, "must not alias"),
    (dict(K=250), 3, "multiple of 32"),
])
def test_qkv_rope_validation(lib, kw, code, msg):
    """dk_gemv_w4a16_qkv_rope rejects bad shapes, tiles, pointers and aliasing before any launch."""
    rc, m = _qkv_rope(lib, **kw)
    assert rc == code and msg in m, (rc, m)


def test_fused_gemv_validation(lib):
    assert _fused(lib, lib.dk_gemv_w4a16_rmsnorm, stage=3)[0] == 4
    assert _fused(lib, lib.dk_gemv_w4a16_rmsnorm, norm_w=None)[0] == 1
    assert _fused(lib, lib.dk_gemv_w4a16_rmsnorm, x_out=A16)[0] == 4
    assert _fused(lib, lib.dk_gemv_w4a16_rmsnorm, pf=4)[0] == 4
    rc, m = _fused(lib, lib.dk_gemv_w4a16_rmsnorm, warps=3, K=4096)     # row groups of 2 waves at K 4096
    assert rc == 3 and "whole row groups" in m
    assert _fused(lib, lib.dk_gemv_w4a16_gate_up, warps=17)[0] == 4


def test_gemv_f16_validation(lib):
    f = lambda **kw: _err(lib, lib.dk_gemv_f16(*dict(dict(R=2, warps=4, pf=2, w=A16, x=A16, y=B16, N=64, K=2048),
                                                      **kw).values(), None))
    assert f(R=3)[0] == 4 and f(warps=3)[0] == 4 and f(pf=4)[0] == 4 and f(N=0)[0] == 3
    assert f(K=2044)[0] == 3 and f(K=4104)[0] == 3 and f(w=A16 + 8)[0] == 2 and f(y=B16 + 1)[0] == 2
    assert f(K=4096, R=4)[0] == 4 and "R <= 2" in f(K=4096, R=4)[1]
    assert f(x=None)[0] == 1
    n = lambda **kw: _err(lib, lib.dk_gemv_f16_rmsnorm(*dict(dict(R=2, warps=4, pf=2, w=A16, x=A16, d=None, nw=A16,
                                                                  eps=1e-5, xo=None, y=B16, N=64, K=2048),
                                                             **kw).values(), None))
    assert n(nw=None)[0] == 1 and n(xo=A16)[0] == 4 and n(d=A16 + 4)[0] == 2 and n(R=8)[0] == 4


def test_small_op_validation(lib):
    assert _err(lib, lib.dk_add_rmsnorm(A16, None, A16, A16, 2047, 1e-5, None))[0] == 3
    rc, m = _err(lib, lib.dk_add_rmsnorm(A16, None, A16, A16, 65544, 1e-5, None))     # two-pass row: no aliasing
    assert rc == 4 and "must not alias" in m
    assert _err(lib, lib.dk_add_rmsnorm(A16, B16, A16 + 4096, B16, 65544, 1e-5, None))[0] == 4  # out == delta
    assert _err(lib, lib.dk_add_rmsnorm(A16 + 2, None, A16, A16, 2048, 1e-5, None))[0] == 2
    assert _err(lib, lib.dk_add_rmsnorm(A16, A16 + 8, A16, A16, 2048, 1e-5, None))[0] == 2
    assert _err(lib, lib.dk_add_rmsnorm(None, None, A16, A16, 2048, 1e-5, None))[0] == 1
    assert _err(lib, lib.dk_swiglu(A16, A16, 5630, None))[0] == 3
    assert _err(lib, lib.dk_swiglu(A16, A16 + 4, 5632, None))[0] == 2
    rope = lambda **kw: _err(lib, lib.dk_rope_append(*dict(
        dict(qkv=A16, c=A16, s=A16, pos=A16, bt=A16, kc=A16, vc=A16, n_q=32, n_kv=4, D=64, page=16, max_pos=100,
             n_pages=8, n_bt=8), **kw).values(), None))
    assert rope(D=80)[0] == 3 and rope(page=10)[0] == 4 and rope(max_pos=0)[0] == 3 and rope(bt=None)[0] == 1
    assert _err(lib, lib.dk_argmax_advance(A16, 0, A16, A16, None))[0] == 3
    assert _err(lib, lib.dk_argmax_advance(None, 10, A16, A16, None))[0] == 1
    assert _err(lib, lib.dk_argmax_advance_split(A16, 0, A16, A16, A16, None))[0] == 3
    assert _err(lib, lib.dk_argmax_advance_split(A16, 10, A16, A16, None, None))[0] == 1
    assert _err(lib, lib.dk_argmax_advance_split(A16, 10, A16, A16, A16 + 4, None))[0] == 2
    q = lambda **kw: _err(lib, lib.dk_quantize_w4(*dict(dict(w=A16, p=A16, sz=A16, N=4, K=256, G=128, clip=0),
                                                        **kw).values(), None))
    assert q(G=1024)[0] == 4 and q(G=48)[0] == 4 and q(K=192)[0] == 3 and q(w=A16 + 2)[0] == 2
    assert q(clip=2)[0] == 4
    bw = lambda **kw: _err(lib, lib.dk_bw_read(*dict(dict(buf=A16, n=1024, sink=A16, words=4, blocks=4, threads=256,
                                                         unroll=4), **kw).values(), None))
    assert bw(unroll=3)[0] == 4 and bw(unroll=32)[0] == 4 and bw(buf=A16 + 1)[0] == 2 and bw(sink=A16 + 2)[0] == 2
    assert bw(threads=96)[0] == 3 and bw(threads=2048)[0] == 3 and bw(blocks=0)[0] == 3 and bw(words=0)[0] == 3
    assert bw(blocks=(1 << 22) + 1)[0] == 3
    assert bw(n=8)[0] == 3 and bw(sink=None)[0] == 1 and bw(buf=None)[0] == 1


def test_prefill_validation(lib):
    g = lambda **kw: _err(lib, lib.dk_gemm_w4a16(*dict(dict(p=A16, sz=A16, x=A16, y=B16, M=64, N=128, K=256, G=128,
                                                            epi=0), **kw).values(), None))
    assert g(K=240)[0] == 3 and g(K=288, G=96)[0] == 4 and g(G=16)[0] == 4 and g(epi=2)[0] == 4
    assert g(epi=1, N=127)[0] != 0 and g(y=A16)[0] == 4 and g(x=None)[0] == 1 and g(M=0)[0] == 3
    # split-K workspace: the bytes a shape needs (fp32 partials [S, M, N]; 0 where it does not split), then every
    # workspace check ahead of a launch
    wb = lib.dk_gemm_w4a16_workspace_bytes
    assert wb(512, 4096, 14336, 128, 0) == 4 * 512 * 4096 * 4 and wb(512, 2048, 5632, 128, 0) == 2 * 512 * 2048 * 4
    assert wb(512, 4096, 4096, 128, 0) == 0      # an unsplit tiling fills the CUs and K is short: no split
    assert wb(512, 2560, 2048, 128, 0) == 0 and wb(512, 2048, 2048, 128, 0) == 0   # splits under 16 chunks
    assert wb(512, 4096, 4096, 128, 1) == 0 and wb(512, 28672, 4096, 128, 0) == 0 and wb(512, 4096, 4096, 32, 0) == 0
    assert wb(32, 4096, 4096, 128, 0) == 0 and wb(512, 4096, 4100, 128, 0) == 0 and wb(0, 4096, 4096, 128, 0) == 0
    need = wb(512, 4096, 14336, 128, 0)
    W = 0x7f0000000000
    ws = lambda **kw: _err(lib, lib.dk_gemm_w4a16_ws(*dict(dict(
        p=A16, sz=A16, x=A16, y=B16, M=512, N=4096, K=14336, G=128, epi=0, w=W, wbytes=need), **kw).values(), None))
    assert ws(wbytes=need - 1)[0] == 3 and "needs %d" % need in ws(wbytes=need - 1)[1]
    assert ws(w=W + 8)[0] == 2 and ws(w=B16 - 64)[0] == 4 and ws(w=A16)[0] == 4
    assert ws(K=240)[0] == 3 and ws(x=None)[0] == 1
    # epilogue 2: the split partials alone, only where the shape splits (y unused)
    assert wb(512, 4096, 14336, 128, 2) == need
    assert ws(epi=2, K=4096, wbytes=1 << 30)[0] == 4 and "splits" in ws(epi=2, K=4096, wbytes=1 << 30)[1]
    assert ws(epi=2, wbytes=need - 1)[0] == 3 and ws(epi=2, w=None)[0] == 1
    rp = lambda **kw: _err(lib, lib.dk_rmsnorm_rows_parts(*dict(dict(
        x=A16, p=W, S=2, ps=4 * 2048, w=A16, xo=A16, out=B16, M=4, H=2048, eps=1e-5), **kw).values(), None))
    assert rp(S=0)[0] == 3 and rp(S=65)[0] == 3 and rp(ps=2046)[0] == 3 and rp(ps=1024)[0] == 3
    assert rp(H=2044)[0] == 3 and rp(M=0)[0] == 3 and rp(p=W + 4)[0] == 2 and rp(out=A16)[0] == 4
    assert rp(p=None)[0] == 1 and rp(p=B16 - 4 * 2048)[0] == 4 and "overlap" in rp(p=B16 - 4 * 2048)[1]
    rr = lambda **kw: _err(lib, lib.dk_rope_append_rows(*dict(
        dict(qkv=A16, c=A16, s=A16, pos=A16, bt=A16, kc=A16, vc=A16, M=8, n_q=32, n_kv=4, D=64, page=16, max_pos=100,
             n_pages=8, n_bt=8), **kw).values(), None))
    assert rr(M=0)[0] == 3 and rr(M=70000)[0] == 3 and rr(D=96)[0] == 3 and rr(page=12)[0] == 4
    assert rr(vc=None)[0] == 1 and rr(n_bt=0)[0] == 3
    nr = lambda **kw: _err(lib, lib.dk_rmsnorm_rows(*dict(dict(x=A16, rows=None, ns=4, d=None, w=A16, xo=A16, out=B16,
                                                               M=4, H=2048, eps=1e-5), **kw).values(), None))
    assert nr(H=2044)[0] == 3 and nr(H=65544)[0] == 3 and nr(M=0)[0] == 3 and nr(out=A16)[0] == 4
    assert nr(d=A16 + 2)[0] == 2
    assert nr(rows=A16 + 4)[0] == 2 and nr(rows=A16)[0] == 4 and nr(w=None)[0] == 1
    assert nr(ns=5)[0] == 3 and nr(rows=A16, xo=B16 + 0x1000, ns=0)[0] == 3 and "n_src" in nr(ns=3)[1]
    ap = lambda **kw: _err(lib, lib.dk_attention_prefill(*dict(
        dict(qkv=A16, pos=A16, bt=A16, n_bt=8, kc=A16, vc=A16, n_pages=8, page=16, n_q=32, n_kv=4, D=64, M=8,
             max_ctx=128, out=B16), **kw).values(), None))
    assert ap(n_q=24, n_kv=8)[0] == 3 and ap(n_q=64, n_kv=4)[0] == 3 and ap(D=80)[0] == 3 and ap(M=0)[0] == 3
    assert ap(page=24)[0] == 4 and ap(max_ctx=0)[0] == 4 and ap(qkv=A16 + 2)[0] == 2
    assert "max_ctx must be >= 1" in ap(max_ctx=-3)[1] and ap(out=None)[0] == 1


def test_error_message_is_cleared_per_thread(lib):
    lib.dk_swiglu(A16, A16, 3, None)
    assert "multiple of 8" in lib.dk_last_error().decode()


def test_shim_rejects_cpu_tensors(lib):
    K = ext.DecodeKernels(lib)
    packed = torch.zeros(4, 16, dtype=torch.int32)
    sz = torch.zeros(4, 1, 2, dtype=torch.half)
    with pytest.raises(RuntimeError, match="must be a contiguous CUDA tensor"):
        K.gemv_w4a16(2, 4, 0, 0, packed, sz, torch.zeros(128, dtype=torch.half), torch.zeros(4, dtype=torch.half),
                     128)
    with pytest.raises(RuntimeError, match="must be a contiguous CUDA tensor"):
        K.swiglu(torch.zeros(16, dtype=torch.half), torch.zeros(8, dtype=torch.half))


def _qkv_rope_args(**kw):
    """CPU tensors of consistent shapes for the qkv RoPE shim (n_q 4, n_kv 2, head_dim 64, K 256, G 128)."""
    n_q, n_kv, D, K, G = 4, 2, 64, 256, 128
    N = (n_q + 2 * n_kv) * D
    h = dict(dtype=torch.half)
    a = dict(stage=4, R=2, warps=0, pf=0, packed=torch.zeros(N, K // 8, dtype=torch.int32),
             sz=torch.zeros(N, K // G, 2, **h), x=torch.zeros(K, **h), row=None, delta=torch.zeros(K, **h),
             norm_w=torch.ones(K, **h), eps=1e-5, x_out=torch.zeros(K, **h), qkv=torch.zeros(N, **h),
             cos_t=torch.zeros(64, D // 2), sin_t=torch.zeros(64, D // 2), pos=torch.zeros(1, dtype=torch.int32),
             bt=torch.zeros(4, dtype=torch.int32), kc=torch.zeros(4, n_kv, 16, D, **h),
             vc=torch.zeros(4, n_kv, 16, D, **h), n_q=n_q, n_kv=n_kv, group=G)
    a.update(kw)
    return a


@pytest.mark.parametrize("kw,msg", [
    ({}, "must be a contiguous CUDA tensor"),                      # consistent: only the device check is left
    ({"sz": torch.zeros(512, 1, 2, dtype=torch.half)}, "shape mismatch"),
    ({"group": 64}, "shape mismatch"),                              # sz groups disagree with K / group
    ({"packed": torch.zeros(512, 32, dtype=torch.int16)}, "int32"),
    ({"qkv": torch.zeros(500, dtype=torch.half)}, "qkv as many values"),
    ({"sin_t": torch.zeros(32, 32)}, "cos_t and sin_t"),
    ({"cos_t": torch.zeros(64, 16)}, "cos_t and sin_t"),
    ({"x": torch.zeros(255, dtype=torch.half)}, "x must hold K values"),
    ({"x": torch.zeros(256)}, "x must be torch.float16"),
    ({"row": torch.zeros(1, dtype=torch.int32), "delta": None, "x": torch.zeros(10, 256, dtype=torch.half)},
     "int64 index"),
    ({"row": torch.zeros(1, dtype=torch.int64), "x": torch.zeros(10, 256, dtype=torch.half)}, "no delta"),
    ({"row": torch.zeros(1, dtype=torch.int64), "delta": None, "x": torch.zeros(256, dtype=torch.half)},
     "int64 index"),
    ({"delta": torch.zeros(128, dtype=torch.half)}, "delta must be fp16 \\[K\\]"),
    ({"x_out": torch.zeros(256)}, "x_out must be fp16 \\[K\\]"),
    ({"norm_w": torch.ones(128, dtype=torch.half)}, "norm_w must be fp16 \\[K\\]"),
    ({"norm_w": None}, "without norm_w"),
    ({"vc": torch.zeros(4, 2, 16, 128, dtype=torch.half)}, "cache must be"),
    ({"n_kv": 1}, "cache must be"),
    ({"pos": torch.zeros(1, dtype=torch.int64)}, "pos must be torch.int32"),
    ({"bt": torch.zeros(4, dtype=torch.int64)}, "bt must be torch.int32"),
    ({"pos": torch.zeros(0, dtype=torch.int32)}, "pos must hold"),
])
def test_qkv_rope_shim_checks_every_argument(lib, kw, msg):
    """The torch shim of dk_gemv_w4a16_qkv_rope rejects each inconsistent argument with its own message before any
    launch (shape and dtype checks run ahead of the device check, so they are reachable with CPU tensors)."""
    K = ext.DecodeKernels(lib)
    with pytest.raises(RuntimeError, match=msg):
        K.gemv_w4a16_qkv_rope(*_qkv_rope_args(**kw).values())


def test_load_without_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        ext.open_library(tmp_path / "missing.so")


def test_model_rejects_ref_backend():
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape
    with pytest.raises(ValueError, match="oracle.decode_ref"):
        Model({}, LlamaShape(128, 1, 2, 1, 256, 64), DecodeConfig(backend="ref", device="cpu"))


@pytest.mark.parametrize("extra,exc,msg", [
    (dict(attention_bias=True), NotImplementedError, "projection biases"),
    (dict(mlp_bias=True), NotImplementedError, "projection biases"),
    (dict(hidden_act="gelu"), NotImplementedError, "silu only"),
    (dict(rope_parameters={"rope_theta": 5e5, "rope_type": "llama3", "factor": 8.0}), NotImplementedError, "llama3"),
    (dict(head_dim=96), ValueError, "head_dim"),
])
def test_model_rejects_unsupported_configs(extra, exc, msg):
    """Configurations outside the Llama composition the kernels implement are refused before any weight is read,
    instead of running with parts of the model silently dropped."""
    import types
    from runtime.model import DecodeConfig, Model
    c = types.SimpleNamespace(hidden_size=128, num_hidden_layers=1, num_attention_heads=2, num_key_value_heads=1,
                              intermediate_size=256, vocab_size=64, rms_norm_eps=1e-5, **extra)
    with pytest.raises(exc, match=msg):
        Model({}, c, DecodeConfig(device="cpu"))
