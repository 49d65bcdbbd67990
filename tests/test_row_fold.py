"""The transposed row fold of the row-tile GEMV (fold_lane / fold_rows / fold_finish in csrc/common.hpp), simulated
lane by lane on the CPU: after the merging steps every lane of each 16-lane DPP row holds the sum over that DPP row
of a different row, the lanes the kernel lets write cover each row once, and the quarters summed in LDS give every
row's total over the 64 lanes. The expected sums are formed directly from the lane partials (brute force), so a
wrong c_s formula, partner permutation or merge order fails here. The GPU tests compare the compiled kernels with
the oracle and with each other (tests/test_kernels_gpu.py)."""
import numpy as np
import pytest

# DPP partner of each step within a 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
PARTNER = {
    1: lambda i: i ^ 1,
    2: lambda i: i ^ 2,
    3: lambda i: (i & ~7) | (7 - (i & 7)),
    4: lambda i: (i & ~15) | (15 - (i & 15)),
}


def fold_lane(lane, n):
    b = [(lane >> k) & 1 for k in range(4)]
    c = [b[0] ^ b[2], b[1] ^ b[2], b[2] ^ b[3], b[3]]
    m = sum(1 << s for s in range(4) if (1 << (s + 1)) <= n and c[s])
    return c, m


def dpp(vals, step):
    """vals: per-lane values (64); returns the value each lane reads from its step partner."""
    return np.array([vals[PARTNER[step](i)] for i in range(64)], dtype=vals.dtype)


def simulate(partials, T, NT):
    """partials [64 lanes, n rows] -> the LDS rows [4 quarters, n] the kernel writes, following fold_rows' schedule."""
    n = T * NT
    lanes = [fold_lane(l, n) for l in range(64)]
    p = partials.astype(np.int64).copy()          # p[lane, slot]
    for t in range(NT):
        r0 = t * T
        for s in range(1, 5):
            blk = 1 << s
            if blk > n:
                continue
            half = blk >> 1
            for b in range(0, n, blk):
                end = b + blk - 1
                if r0 <= end < r0 + T:
                    c = np.array([lanes[l][0][s - 1] for l in range(64)])
                    keep = np.where(c == 1, p[:, b + half], p[:, b])
                    send = np.where(c == 1, p[:, b], p[:, b + half])
                    p[:, b] = keep + dpp(send, s)
    for s in range(1, 5):                         # fold_finish: plain steps past the merging ones
        if n < (1 << s):
            p[:, 0] = p[:, 0] + dpp(p[:, 0], s)
    lds = np.full((4, n), np.iinfo(np.int64).min, dtype=np.int64)
    for l in range(64):
        if (l & 15) < min(n, 16):
            m = lanes[l][1]
            for j in range((n + 15) // 16):
                assert lds[l >> 4, 16 * j + m] == np.iinfo(np.int64).min, "two lanes write one row"
                lds[l >> 4, 16 * j + m] = p[l, 16 * j]
    return lds


@pytest.mark.parametrize("T,NT", [(1, 1), (2, 1), (1, 2), (2, 2), (4, 1), (1, 8), (2, 4), (4, 4), (2, 8), (8, 2),
                                  (4, 8), (8, 8), (1, 4), (8, 1)])
def test_fold_gives_every_row_sum(T, NT):
    rng = np.random.default_rng(T * 100 + NT)
    n = T * NT
    partials = rng.integers(-1000, 1000, size=(64, n))
    lds = simulate(partials, T, NT)
    want = partials.reshape(4, 16, n).sum(axis=1)        # per quarter (16-lane DPP row), per row
    assert np.array_equal(lds, want)
    assert np.array_equal(lds.sum(axis=0), partials.sum(axis=0))


def test_lane_rows_are_a_permutation_per_dpp_row():
    for n in (1, 2, 4, 8, 16, 32, 64):
        ms = sorted(fold_lane(l, n)[1] for l in range(16) if l < min(n, 16))
        assert ms == list(range(min(n, 16)))
        # partners of a merging step differ in exactly that step's bit c_s
        for s in range(1, 5):
            if (1 << s) > n:
                continue
            for l in range(64):
                c, _ = fold_lane(l, n)
                cp, _ = fold_lane(PARTNER[s](l), n)
                assert [a ^ b for a, b in zip(c, cp)] == [int(k == s - 1) for k in range(4)]
