"""GPU parity of the fused decode attention (dk_attention_decode) against the oracle's composition of the two reference
ops it replaces: rope_append_ref (reference/ref_ops.py:44-53) then paged_attention_ref (reference/ref_ops.py:76-78)
on the same seeded inputs. Output within the reference's attention tolerance (2e-3 normwise, tests/test_kernels.py:121);
the k / v written into the cache bit-exact (the reference's rope tests hold the v copy at tol 0.0 and the oracle's
rotation is elementwise fp32, reproduced exactly); qkv left untouched."""
import pytest
import torch

from helpers import DEV, assert_close, gen, make_cache
from oracle import ref_ops as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


MODES = ("block", "lean")   # impl 1, impl 3
IMPL = {"block": 1, "lean": 3}


def lean_fits(PS, page, D):
    """impl 3: pages of >= 16 tokens, part sizes a multiple of 16 up to 512 (256 at head_dim 128)."""
    return page >= 16 and PS % 16 == 0 and PS <= (256 if D == 128 else 512)


def run_fused(K, qkv, cos, sin, kc, vc, bt, pos, n_q, n_kv, PS, max_splits, mode="block"):
    """A part size the lean kernel cannot take is checked to be rejected; then None is returned."""
    D = kc.shape[-1]
    if mode == "lean" and not lean_fits(PS, kc.shape[2], D):
        with pytest.raises(RuntimeError, match="impl 3 needs pages"):
            K.attention_decode(qkv, cos, sin, torch.tensor([pos], dtype=torch.int32, device=DEV), bt, kc, vc, n_q,
                               n_kv, PS, torch.empty(n_q, max_splits, D, device=DEV),
                               torch.empty(n_q, max_splits, device=DEV), torch.empty(n_q, max_splits, device=DEV),
                               torch.empty(n_q, D, dtype=torch.half, device=DEV), impl=3)
        return None, None, None
    o_part = torch.full((n_q, max_splits, D), 7.0, device=DEV)
    m_part = torch.full((n_q, max_splits), 7.0, device=DEV)
    l_part = torch.full((n_q, max_splits), 7.0, device=DEV)
    out = torch.zeros(n_q, D, dtype=torch.half, device=DEV)
    K.attention_decode(qkv, cos, sin, torch.tensor([pos], dtype=torch.int32, device=DEV), bt, kc, vc, n_q, n_kv, PS,
                       o_part, m_part, l_part, out, impl=IMPL[mode])
    return out, o_part, m_part


def reference(qkv, cos, sin, kc, vc, bt, pos, n_q, n_kv, D, page, attend=None):
    kr, vr = kc.clone(), vc.clone()
    q = R.rope_append_ref(qkv.clone(), cos, sin, pos, kr, vr, bt, n_q, n_kv, D, page)
    ctx = pos + 1 if attend is None else attend
    return R.paged_attention_ref(q, kr, vr, bt, ctx, page), kr, vr


CASES = [(64, 32, 4), (64, 8, 8), (64, 16, 4), (64, 8, 4), (128, 32, 8), (128, 64, 8), (128, 16, 8), (128, 8, 8)]


@pytest.mark.parametrize("D,n_q,n_kv", CASES)
@pytest.mark.parametrize("ctx", (1, 2, 17, 64, 65, 500, 2048))
@pytest.mark.parametrize("mode", MODES)
def test_fused_attention_matches_rope_then_attention(K, D, n_q, n_kv, ctx, mode):
    page = 16
    theta = 1e4 if D == 64 else 5e5
    cos, sin = R.rope_tables(ctx + 8, D, theta)
    kc, vc, bt = make_cache(ctx, n_kv, page, D=D, peaky=2.0, seed=ctx + D)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(ctx * 3 + n_q)).half()
    ref, kr, vr = reference(qkv, cos, sin, kc, vc, bt, ctx - 1, n_q, n_kv, D, page)
    for PS in sorted({16, 64, 256, ctx}):
        ms = -(-ctx // PS)
        kd, vd, qd = kc.to(DEV), vc.to(DEV), qkv.to(DEV)
        out, _, _ = run_fused(K, qd, cos.to(DEV), sin.to(DEV), kd, vd, bt.to(DEV), ctx - 1, n_q, n_kv, PS, ms,
                              mode)
        if out is None:
            continue
        assert_close(out, ref, 2e-3, f"fused D{D} {n_q}/{n_kv} ctx{ctx} PS{PS} {mode}")
        assert torch.equal(kd.cpu(), kr) and torch.equal(vd.cpu(), vr), f"cache append D{D} ctx{ctx} PS{PS}"
        assert torch.equal(qd.cpu(), qkv), "qkv must not be modified"


@pytest.mark.parametrize("ctx", (100, 1000, 4096))
@pytest.mark.parametrize("mode", MODES)
def test_fused_attention_spare_splits_untouched(K, ctx, mode):
    """Grid sized for more splits than ctx needs (the runtime's cap): partials past the live splits stay untouched."""
    D, n_q, n_kv, page, PS, spare = 64, 32, 4, 16, 64, 7
    cos, sin = R.rope_tables(ctx + 8, D)
    kc, vc, bt = make_cache(ctx + spare * PS, n_kv, page, D=D, seed=ctx)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(ctx)).half()
    ref, _, _ = reference(qkv, cos, sin, kc, vc, bt, ctx - 1, n_q, n_kv, D, page)
    live = -(-ctx // PS)
    out, o_part, m_part = run_fused(K, qkv.to(DEV), cos.to(DEV), sin.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                       ctx - 1, n_q, n_kv, PS, live + spare, mode)
    assert_close(out, ref, 2e-3, f"spare ctx{ctx}")
    assert torch.all(o_part[:, live:] == 7.0) and torch.all(m_part[:, live:] == 7.0)


@pytest.mark.parametrize("mode", MODES)
def test_fused_attention_cap_below_position(K, mode):
    """pos beyond max_splits * PS: the new k / v are still appended (by the last live split) and attention covers the
    first max_splits * PS tokens, as rope_append + paged_attention with the same split buffers do."""
    D, n_q, n_kv, page, PS, ms, pos = 64, 32, 4, 16, 32, 4, 200
    cos, sin = R.rope_tables(pos + 8, D)
    kc, vc, bt = make_cache(pos + 1, n_kv, page, D=D, seed=5)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(5)).half()
    ref, kr, vr = reference(qkv, cos, sin, kc, vc, bt, pos, n_q, n_kv, D, page, attend=ms * PS)
    kd, vd = kc.to(DEV), vc.to(DEV)
    out, _, _ = run_fused(K, qkv.to(DEV), cos.to(DEV), sin.to(DEV), kd, vd, bt.to(DEV), pos, n_q, n_kv, PS, ms,
                          mode)
    assert_close(out, ref, 2e-3, "cap")
    assert torch.equal(kd.cpu(), kr) and torch.equal(vd.cpu(), vr)


@pytest.mark.parametrize("mode", MODES)
def test_fused_attention_position_outside_table_is_noop(K, mode):
    D, n_q, n_kv = 64, 32, 4
    cos, sin = R.rope_tables(64, D)
    kc, vc, bt = make_cache(80, n_kv, 16, D=D, seed=8)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(8)).half()
    kd = kc.to(DEV)
    out, o_part, _ = run_fused(K, qkv.to(DEV), cos.to(DEV), sin.to(DEV), kd, vc.to(DEV), bt.to(DEV), 64, n_q,
                               n_kv, 16, 5, mode)
    assert torch.equal(kd.cpu(), kc) and torch.all(out == 0) and torch.all(o_part == 7.0)


@pytest.mark.parametrize("mode", MODES)
def test_fused_attention_graph_replays(K, mode):
    """One captured launch replayed at several positions (the graph reads *pos anew), eager work between replays;
    every replay equals the eager result."""
    D, n_q, n_kv, page, PS, ms = 64, 32, 4, 16, 32, 10
    cap = PS * ms
    cos, sin = (t.to(DEV) for t in R.rope_tables(cap + 1, D))
    kc0, vc0, bt = (t.to(DEV) for t in make_cache(cap, n_kv, page, D=D, seed=21))
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen(22)).half().to(DEV)
    kc, vc = kc0.clone(), vc0.clone()
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    o_part = torch.empty(n_q, ms, D, device=DEV)
    m_part = torch.empty(n_q, ms, device=DEV)
    l_part = torch.empty_like(m_part)
    out = torch.empty(n_q, D, dtype=torch.half, device=DEV)

    def body():
        K.attention_decode(qkv, cos, sin, pos, bt, kc, vc, n_q, n_kv, PS, o_part, m_part, l_part, out,
                           impl=IMPL[mode])

    expected = {}
    for p in (0, 31, 32, 150, 319):
        kc.copy_(kc0)
        vc.copy_(vc0)
        pos.fill_(p)
        body()
        torch.cuda.synchronize()
        expected[p] = (out.clone(), kc.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for rep in range(3):
        for p in (0, 31, 32, 150, 319):
            kc.copy_(kc0)
            vc.copy_(vc0)
            pos.fill_(p)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, expected[p][0]) and torch.equal(kc, expected[p][1]), (rep, p)
            _ = (qkv.float() * 2).sum().item()
