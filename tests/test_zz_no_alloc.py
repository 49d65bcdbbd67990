"""dk_paged_attention_noalloc: the paged attention op with its split partials in the library's per-device scratch
array instead of caller buffers (for callers that cannot allocate). Checked through the C ABI against the existing
entry point dk_paged_attention on the same inputs -- the same kernels, so the outputs must be bit-identical -- on two
calls in a row, the second with a smaller input (the scratch keeps the first call's partials), and against the
oracle within the attention tolerance; sizes beyond the scratch array are rejected before any launch."""

import pytest
import torch

from helpers import DEV, assert_close, gen, make_cache
from oracle import ref_ops as R
from runtime import ext

A16 = 0x10000


@pytest.fixture(scope="module")
def lib():
    return ext.open_library()


def test_noalloc_rejects_oversized_partials(lib):
    """Sizes whose partials exceed the scratch array fail with DK_ERR_SHAPE and a message, before any HIP call."""
    cap = ext.load().lib.dk_paged_attention_noalloc_bytes
    n_q, D = 64, 128
    splits = 1
    while cap(n_q, D, splits) <= (4 << 20):
        splits *= 2
    rc = lib.dk_paged_attention_noalloc(5, A16, A16, A16, A16, A16, n_q, 8, D, 16, 8, 8, 16, splits, A16, None)
    assert rc == 3 and "scratch array" in lib.dk_last_error().decode()
    assert cap(n_q, D, splits // 2) <= (4 << 20) < cap(n_q, D, splits)
    assert cap(32, 64, 16) == 32 * 16 * 64 * 4 + 2 * 2048 and cap(0, 64, 4) == 0


def _inputs(ctx, n_q, n_kv, D, page, seed):
    kc, vc, bt = make_cache(ctx, n_kv, page, D=D, seed=seed)
    q = torch.randn(n_q, D, generator=gen(seed + 1)).half()
    return q, kc, vc, bt


@pytest.mark.gpu
def test_noalloc_matches_caller_buffer_entry_point_twice():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K = ext.load()
    for call, (ctx, n_q, n_kv, D, PS, ver) in enumerate(((1000, 32, 4, 64, 32, 5), (100, 32, 8, 128, 16, 5))):
        print(f"noalloc call {call}: ctx {ctx} heads {n_q}/{n_kv} D {D} part {PS} version {ver}", flush=True)
        q, kc, vc, bt = _inputs(ctx, n_q, n_kv, D, 16, seed=40 + call)
        S = (ctx + PS - 1) // PS
        qd, kd, vd, btd = q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV)
        pos = torch.tensor([ctx - 1], dtype=torch.int32, device=DEV)
        want = torch.empty(n_q, D, dtype=torch.half, device=DEV)
        K.paged_attention(qd, kd, vd, btd, pos, PS, torch.empty(n_q, S, D, device=DEV),
                          torch.empty(n_q, S, device=DEV), torch.empty(n_q, S, device=DEV), want, ver)
        got = torch.full((n_q, D), float("nan"), dtype=torch.half, device=DEV)
        K.paged_attention_noalloc(qd, kd, vd, btd, pos, PS, S, got, ver)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}: noalloc differs from the caller-buffer entry point"
        assert_close(got, R.paged_attention_ref(q, kc, vc, bt, ctx, 16), 2e-3, f"call {call} vs oracle")
