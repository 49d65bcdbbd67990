#!/usr/bin/env python3
"""Benchmark of the batch-1 W4A16 decode hot path on one MI355X; prints ONE JSON line.

Workload: TinyLlama-1.1B-architecture decode step, random init W ~ N(0, 0.02) quantized W4A16
group 128 on the GPU, 22 layers, hidden 2048, 32 q / 4 kv heads, head_dim 64, SwiGLU 5632, vocab 32000 fp16 LM head,
batch 1, paged KV (page 16), the whole step captured as one hipGraph and replayed per token. A "step" is one token.
`value` = tokens/s over the K timed replays starting at context --ctx (default 512), bracketed by device syncs.

Also measured in the same run:
  * roofline of the dominant kernel, the W4A16 GEMV, at the BASELINE target shape 4096 x 14336 (G128): algorithmic
    bytes per launch (packed + scale/zero + x + y = 31,232,000 B) / mean launch duration from HIP events on the launch
    stream, weights rotated over enough copies (> 1 GiB) that every launch reads from HBM, not L2 or the MALL;
  * the 14336 x 4096 GEMV the same way, and the decode step against its bytes-per-token roofline;
  * cpu_baseline: the CPU oracle's decode step (oracle.decode_ref, the reference's backend="ref" composition on the
    host cores, torch fp32 matvec) on the same weights, a bounded sample of tokens.
"""
import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "llm-decode-kernels_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "W4A16 GEMV HBM GB/s (% of peak) + batch-1 decode tokens/s, TinyLlama shape"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_leg(K, N, Kd, G=128, iters=60, copies=None):
    """Mean / median per-launch duration (us) of the configured W4A16 GEMV with cold weights."""
    import torch
    from oracle import quant_ref as Q
    from runtime.model import default_gemv_config
    from runtime.quant import quantize_pack

    nbytes = Q.gemv_bytes(N, Kd, G)
    copies = copies or max(4, int((1.25 * 2 ** 30) // nbytes) + 1)
    g = torch.Generator(device="cuda").manual_seed(N + Kd)
    w = torch.randn(N, Kd, generator=g, device="cuda") * 0.02
    packed, sz = quantize_pack(w.half(), G)
    del w
    ws = [(packed.clone(), sz.clone()) for _ in range(copies)]
    x = torch.randn(Kd, generator=g, device="cuda").half()
    y = torch.empty(N, dtype=torch.half, device="cuda")
    cfg = default_gemv_config(N, Kd)
    for i in range(copies):
        K.gemv_w4a16(*cfg, ws[i][0], ws[i][1], x, y, G)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for i, (s, e) in enumerate(ev):
        p, z = ws[i % copies]
        s.record()
        K.gemv_w4a16(*cfg, p, z, x, y, G)
        e.record()
    torch.cuda.synchronize()
    t = [s.elapsed_time(e) * 1e3 for s, e in ev]
    return {"N": N, "K": Kd, "group": G, "cfg": list(cfg), "bytes": nbytes, "mean_us": statistics.mean(t),
            "median_us": statistics.median(t), "min_us": min(t), "copies": copies,
            "gbps_mean": nbytes / statistics.mean(t) / 1e3, "gbps_median": nbytes / statistics.median(t) / 1e3}


def decode_leg(model, ctx, steps, warmup):
    import torch
    model.reset(ctx)
    for _ in range(warmup):
        model.run_step()
    torch.cuda.synchronize()
    model.reset(ctx)
    per = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in per:
        s.record()
        model.run_step()
        e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tok_us = sorted(s.elapsed_time(e) * 1e3 for s, e in per)
    total_us = sum(tok_us)
    return {"ctx_start": ctx, "steps": steps, "ms_per_step": total_us / steps / 1e3, "tok_s": steps / (total_us / 1e6),
            "median_us": statistics.median(tok_us), "p10_us": tok_us[len(tok_us) // 10],
            "p90_us": tok_us[(9 * len(tok_us)) // 10], "wall_tok_s": steps / wall}


def cpu_baseline_leg(model, shape, ctx, budget_s=20.0, max_tokens=8):
    """Tokens/s of the CPU oracle decode step on the host cores (a bounded sample)."""
    import torch
    from __graft_entry__ import _ref_weights
    from oracle.decode_ref import RefDecoder

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(cores)
    dec = RefDecoder(_ref_weights(model, shape), shape, max_ctx=ctx + max_tokens + 2, page=model.cfg.page,
                     block_table=torch.arange((ctx + max_tokens + 2) // model.cfg.page + 2, dtype=torch.int32))
    dec.step(1, ctx)                                   # warm-up (first-touch of the weights)
    n, t0 = 0, time.perf_counter()
    while n < max_tokens and (time.perf_counter() - t0) < budget_s:
        dec.step(1 + n, ctx + 1 + n)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} TinyLlama decode steps of oracle.decode_ref (torch fp32 CPU, reference backend='ref' "
                      f"composition) at ctx {ctx}, after 1 warm-up step, {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--gemv-iters", type=int, default=60)
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only (the batch-1 decode path is single-GPU by design); got --gpus {a.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from runtime import ext
    from runtime.model import DecodeConfig, Model
    from runtime.synth import TINYLLAMA, SyntheticLlama

    K = ext.load()
    dev_name = torch.cuda.get_device_properties(0).name
    log(f"device {dev_name}; building TinyLlama-shape W4A16 model")
    t0 = time.perf_counter()
    cap = a.ctx + a.steps + a.warmup + 16
    cfg = DecodeConfig(lm_head="fp16", max_ctx=cap)
    model = Model(SyntheticLlama(TINYLLAMA, seed=0), TINYLLAMA, cfg)
    model.prepare(cap)
    log(f"model built + graph captured in {time.perf_counter() - t0:.1f}s (part_size {model.part_size}, "
        f"max_splits {model.max_splits})")

    dec = decode_leg(model, a.ctx, a.steps, a.warmup)
    log(f"decode: {dec['tok_s']:.1f} tok/s, median {dec['median_us']:.1f} us/token")
    bpt = model.bytes_per_token(a.ctx + a.steps // 2)
    g1 = gemv_leg(K, 4096, 14336, iters=a.gemv_iters)
    log(f"gemv 4096x14336: mean {g1['mean_us']:.2f} us -> {g1['gbps_mean']:.0f} GB/s")
    g2 = gemv_leg(K, 14336, 4096, iters=a.gemv_iters)
    log(f"gemv 14336x4096: mean {g2['mean_us']:.2f} us -> {g2['gbps_mean']:.0f} GB/s")
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline_leg(model, TINYLLAMA, a.ctx)
        log(f"cpu baseline: {cpu['value']:.3f} tok/s on {cpu['cores']} cores")

    out = {
        "metric": METRIC, "value": round(dec["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(dec["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "w4a16 (fp16 activations, fp32 accumulate)",
        "data": "synthetic (random-init weights N(0,0.02), random token ids)",
        "config": {"workload": "TinyLlama-1.1B-shape W4A16 G128 decode step, fp16 LM head, hipGraph replay",
                   "model": "TinyLlama-1.1B architecture", "global_batch": 1, "seq_len": a.ctx,
                   "parallelism": "single GPU", "device": dev_name},
        "roofline": {"bound": "hbm", "kernel": f"W4A16 GEMV 4096x14336 G128 cfg {g1['cfg']}",
                     "achieved": round(g1["gbps_mean"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g1["gbps_mean"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": g1["bytes"], "mean_us": round(g1["mean_us"], 3),
                     "median_us": round(g1["median_us"], 3)},
        "gemv_14336x4096": {"mean_us": round(g2["mean_us"], 3), "gbps": round(g2["gbps_mean"], 1),
                            "frac": round(g2["gbps_mean"] / HBM_PEAK_GBS, 4), "cfg": g2["cfg"]},
        "decode": {**{k: round(v, 3) if isinstance(v, float) else v for k, v in dec.items()},
                   "bytes_per_token": bpt, "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
                   "frac_of_roofline": round(dec["tok_s"] / (HBM_PEAK_GBS * 1e9 / bpt), 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
