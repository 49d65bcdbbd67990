"""Per-shape W4A16 GEMV tuner for MI355X (the role of the reference's scripts/autotune.py:27-54).

For every (N, K, group) shape, sweeps the kernel family of libdk_amd (stage 2: whole-row waves, R rows per wave x
waves per workgroup x 2^pf steps in flight; stage 3: split-K, R rows per workgroup x waves x one-step prefetch;
stage 4: 2^pf row tiles of R rows over a workgroup that covers K once) with
cold weights (runtime.timing), and writes

    configs/autotune.json   {"device": ..., "best": {"NxK_G": [stage, R, warps, pf]}, "best_tile": {the best stage-4
                             entry}, "us": {"NxK_G": us}, "best_norm": {the fused residual + RMSNorm GEMV},
                             "us_norm": {...}, "grid": [every measurement]}

The runtime (runtime.model.Model.gemv_cfg) reads "best"; 3-element entries [R, warps, pf] of the reference's schema
are read as stage 2. Run:  python -m runtime.autotune [--shapes tinyllama,llama3_8b,baseline] [--groups 128]
"""
import argparse
import json
import pathlib
import sys

import torch

from . import ext
from .quant import quantize_pack
from .timing import ColdCopies, graph_time, n_copies

PKG = pathlib.Path(__file__).resolve().parents[1]
CONFIG = PKG / "configs" / "autotune.json"

SHAPE_SETS = {
    # TinyLlama-1.1B decode: qkv, o, gate|up, down, INT4 LM head
    "tinyllama": {"qkv": (2560, 2048), "o": (2048, 2048), "gate_up": (11264, 2048), "down": (2048, 5632),
                  "lm_head": (32000, 2048)},
    # Llama-3-8B decode
    "llama3_8b": {"qkv8b": (6144, 4096), "o8b": (4096, 4096), "gate_up8b": (28672, 4096), "down8b": (4096, 14336),
                  "lm_head8b": (128256, 4096)},
    # BASELINE config 1 and the standalone target shapes
    "baseline": {"cfg1": (5632, 2048), "w4096x14336": (4096, 14336), "w14336x4096": (14336, 4096)},
}


def candidates(N, K):
    out = []
    for R in (1, 2, 4, 8):
        for w in (1, 2, 4, 8):
            for pf in range(4):
                if (1 << pf) > 16 // R or (1 << pf) > max(1, -(-K // 2048)):
                    continue
                out.append((2, R, w, pf))
    U = K // 32
    full = min(16, -(-U // 64))
    for R in (1, 2, 4, 8):
        for w in sorted({1, 2, 4, 8, full}):
            for pf in (0, 1):
                if pf and U <= 64 * w:
                    continue
                out.append((3, R, w, pf))
    if K <= 32768:
        out += [(4, R, 0, pf) for R in (1, 2, 4, 8) for pf in range(4)]
    return [c for c in out if not (c[0] == 2 and K > 32768)]


def norm_candidates():
    """stage-4 configurations of the fused residual + RMSNorm GEMV (dk_gemv_w4a16_rmsnorm)."""
    return [(4, R, 0, pf) for R in (1, 2, 4, 8) for pf in range(4)]


def tune_norm_shape(Kx, N, K, G, reps=5, log=print):
    """Best configuration of the fused-norm GEMV for one shape, cold weights; also returns the time of the separate
    add_rmsnorm + best plain GEMV pair so the runtime can tell whether fusing pays at this shape."""
    g = torch.Generator(device="cuda").manual_seed(N * 17 + K)
    packed, sz = quantize_pack((torch.randn(N, K, generator=g, device="cuda") * 0.02).half(), G)
    x = torch.randn(K, generator=g, device="cuda").half()
    d = torch.randn(K, generator=g, device="cuda").half()
    w = torch.ones(K, dtype=torch.half, device="cuda")
    xo, nrm = torch.empty_like(x), torch.empty_like(x)
    y = torch.empty(N, dtype=torch.half, device="cuda")
    cold = ColdCopies([packed, sz], n_copies(gemv_bytes(N, K, G)))
    recs = []
    for cfg in norm_candidates():
        _, med = graph_time(lambda i: Kx.gemv_w4a16_rmsnorm(*cfg, *cold[i], x, None, d, w, 1e-5, xo, y, G),
                            cold.copies, reps)
        recs.append({"N": N, "K": K, "G": G, "cfg": list(cfg), "median_us": med, "variant": "rmsnorm"})
    best = min(recs, key=lambda r: r["median_us"])
    log(f"  norm {N}x{K} G{G}: best {best['cfg']} {best['median_us']:.2f} us; {len(recs)} configs")
    del cold
    return best, recs


def gemv_bytes(N, K, G):
    return N * K // 2 + N * (K // G) * 4 + 2 * K + 2 * N


def tune_shape(Kx, N, K, G, reps=5, log=print):
    g = torch.Generator(device="cuda").manual_seed(N * 131 + K)
    packed, sz = quantize_pack((torch.randn(N, K, generator=g, device="cuda") * 0.02).half(), G)
    x = torch.randn(K, generator=g, device="cuda").half()
    y = torch.empty(N, dtype=torch.half, device="cuda")
    nb = gemv_bytes(N, K, G)
    cold = ColdCopies([packed, sz], n_copies(nb))
    recs = []
    for cfg in candidates(N, K):
        mn, med = graph_time(lambda i: Kx.gemv_w4a16(*cfg, *cold[i], x, y, G), cold.copies, reps)
        recs.append({"N": N, "K": K, "G": G, "cfg": list(cfg), "min_us": mn, "median_us": med,
                     "gbps": nb / med / 1e3})
    del cold
    best = min(recs, key=lambda r: r["median_us"])
    log(f"  {N}x{K} G{G}: best {best['cfg']} {best['median_us']:.2f} us {best['gbps']:.0f} GB/s "
        f"({best['gbps'] / 80:.1f}% of 8 TB/s); {len(recs)} configs")
    return best, recs


# GEMVs that consume a residual + RMSNorm in the decode step (qkv, gate|up, INT4 LM head)
NORM_SHAPES = {"tinyllama": ((2560, 2048), (11264, 2048), (32000, 2048)),
               "llama3_8b": ((6144, 4096), (28672, 4096), (128256, 4096)), "baseline": ()}


def tune(shape_sets=("tinyllama", "llama3_8b", "baseline"), groups=(128,), reps=5, path=CONFIG, log=print):
    Kx = ext.load()
    old = json.load(open(path)) if pathlib.Path(path).exists() else {}
    best, us, grid = dict(old.get("best", {})), dict(old.get("us", {})), []
    best_tile = dict(old.get("best_tile", {}))
    best_norm, us_norm = dict(old.get("best_norm", {})), dict(old.get("us_norm", {}))
    for ss in shape_sets:
        for (N, K) in NORM_SHAPES.get(ss, ()):
            for G in groups:
                b, recs = tune_norm_shape(Kx, N, K, G, reps, log)
                key = f"{N}x{K}_G{G}"
                best_norm[key], us_norm[key] = b["cfg"], round(b["median_us"], 3)
                grid += recs
    for ss in shape_sets:
        for name, (N, K) in SHAPE_SETS[ss].items():
            for G in groups:
                b, recs = tune_shape(Kx, N, K, G, reps, log)
                key = f"{N}x{K}_G{G}"
                best[key], us[key] = b["cfg"], round(b["median_us"], 3)
                tiles = [r for r in recs if r["cfg"][0] == 4]
                if tiles:
                    best_tile[key] = min(tiles, key=lambda r: r["median_us"])["cfg"]
                grid += [dict(r, shape=name) for r in recs]
    out = {"device": torch.cuda.get_device_properties(0).name, "best": best, "best_tile": best_tile, "us": us,
           "best_norm": best_norm, "us_norm": us_norm, "grid": grid}
    pathlib.Path(path).parent.mkdir(exist_ok=True)
    json.dump(out, open(path, "w"), indent=1)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default="tinyllama,llama3_8b,baseline")
    ap.add_argument("--groups", default="128")
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--out", default=str(CONFIG))
    a = ap.parse_args(argv)
    tune(a.shapes.split(","), tuple(int(g) for g in a.groups.split(",")), a.reps, a.out,
         log=lambda *s: print(*s, flush=True))


if __name__ == "__main__":
    sys.exit(main())
