#!/usr/bin/env python3
"""Benchmark of the batch-1 W4A16 decode hot path on one MI355X; prints ONE JSON line on stdout.

value: BASELINE config 4, the TinyLlama-1.1B-architecture decode step (random init W ~ N(0, 0.02) quantized W4A16
group 128 on the GPU; 22 layers, hidden 2048, 32 q / 4 kv heads, head_dim 64, SwiGLU 5632, vocab 32000, fp16 LM
head; batch 1; paged KV, page 16), the whole step captured as one hipGraph and replayed once per token. A "step" is
one token. Timed: K replays starting at context --ctx (default 512) after W warm-up replays, bracketed by device
syncs; value = K / elapsed (tokens/s).

Also measured in the same run (extra keys of the JSON line):
  roofline      the dominant kernel, the W4A16 GEMV, at BASELINE's target shape 4096 x 14336 G128 with its tuned
                configuration: algorithmic bytes per launch (packed + scale/zero + x + y = 31,232,000 B) / mean launch
                duration. The duration comes from HIP events around a hipGraph of back-to-back launches on the
                capture stream, each launch reading a different cold copy of the weights (> 2.5 x the 256 MB MALL),
                so every byte comes from HBM. `traffic` is the HBM bytes per launch measured in this run: two
                rocprofv3 counter passes (FETCH_SIZE, then WRITE_SIZE) over `bench.py --leg gemv` in child
                processes, each scaled by what the same counter reads for a plain read / copy of known size in the
                same child (null, with the reason, when rocprofv3 or the counters are unavailable).
  gemv_14336x4096, gemv_cfg1   the other BASELINE GEMV shapes the same way;
  read_ceiling  the library's bw_read streaming the same number of bytes: what a kernel that only reads gets;
  decode        per-token statistics, the bytes-per-token roofline of the step, ctx 2048 as well;
  clocks        shader / memory clock and temperature of the GPU sampled from sysfs while each leg runs (the role of
                the reference's NVML sampling, bench/timing.py:35-49,119-138), so a slow box can be told from a slow
                kernel;
  cpu_baseline  the CPU oracle's decode step (oracle.decode_ref: the reference backend="ref" composition, torch fp32
                matvec) on the host cores: median and IQR of 30 timed steps after 5 warm-up steps, at ctx 512 (the
                value) and at ctx 2048, on the same weights.

--gpus N > 1 exits with a message: the path is single-GPU by design (one GPU per box here).
--leg gemv runs only the GEMV roofline leg (used under rocprofv3 for the kernel trace and counter passes); --leg attn8b
only the Llama-3-8B ctx-4096 attention and bw_read of its K/V bytes (the same, for the attention kernels); --leg
readsweep bw_read from 2 to 512 MB with a fixed-cost + bandwidth fit; --leg decode / prefill / decode8b / kernels run
one leg alone (the decode and prefill legs without the standalone GEMV and kernel legs, so that their traces hold only
the model's kernels).
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
# second TinyLlama decode leg (BASELINE config 4 names contexts 512 and 2048) and the prefill prompt
CTX_LONG, CTX_LONG_STEPS, CTX_LONG_WARMUP = 2048, 64, 8
PREFILL_TOKENS = 512
GEMV_KERNEL = "gemv_w4a16"          # kernel-name substring of the roofline GEMV in counter output


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def leg_caps(ctx, steps, warmup):
    """Context caps of the legs that share one TinyLlama model. A decode leg starts at `ctx`, runs `warmup` steps,
    resets to `ctx` and runs `steps` steps, so its cap is ctx + max(steps, warmup) (+ slack); the model's max_ctx
    covers every cap that a later prepare() asks for, whatever --ctx / --steps / --warmup are."""
    slack = 16
    caps = {"decode": ctx + max(steps, warmup) + slack,
            "decode_long": CTX_LONG + max(CTX_LONG_STEPS, CTX_LONG_WARMUP) + slack,
            "prefill": PREFILL_TOKENS + slack}
    caps["max_ctx"] = max(caps.values())
    return caps


def read_clocks(pci):
    """One clock sample of the GPU at sysfs directory pci (runtime.timing.read_clocks)."""
    from runtime.timing import read_clocks as rc
    return rc(pci)


class ClockSampler:
    """Samples read_clocks every `period` s in a thread while a leg runs; summary() gives per-field min / median /
    max and the sample count (empty when sysfs exposes no clock for this device)."""

    def __init__(self, period=0.02):
        import threading
        from runtime.timing import gpu_sysfs_dir
        self.period, self.samples, self.stop = period, [], threading.Event()
        self.pci = gpu_sysfs_dir()
        self.thread = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        while not self.stop.is_set():
            s = read_clocks(self.pci)
            if s:
                self.samples.append(s)
            self.stop.wait(self.period)

    def __enter__(self):
        if self.pci is not None:
            self.thread.start()
        return self

    def __exit__(self, *exc):
        self.stop.set()
        if self.thread.is_alive():
            self.thread.join()

    def summary(self):
        from runtime.timing import clock_summary
        return clock_summary(self.samples)


def traffic_leg(nbytes, timeout=180):
    """HBM bytes per launch of the roofline GEMV, measured now: rocprofv3 runs `bench.py --leg gemv` twice in a child
    process, once collecting FETCH_SIZE and once WRITE_SIZE (one counter group per pass); each counter is scaled by
    what it reads for the bw_read / copy kernels of known size that the same child runs (runtime.rocprof_summary.pmc).
    Returns (summary dict, None) or (None, reason)."""
    import shutil
    import signal
    import subprocess
    import tempfile
    from runtime import rocprof_summary

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not on PATH"
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="dk_pmc_", dir="/tmp"))
    env = {**os.environ, "TMPDIR": "/tmp"}
    dirs = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tmp / counter.lower()
        cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", str(d), "-o", "pmc", "--",
               sys.executable, str(ROOT / "bench.py"), "--leg", "gemv", "--warm-ms", "2", "--window-ms", "5"]
        log(f"traffic: rocprofv3 --pmc {counter} over bench.py --leg gemv")
        p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE,
                             start_new_session=True)
        try:
            _, err = p.communicate(timeout=timeout)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.communicate()
            return None, f"rocprofv3 --pmc {counter} did not finish in {timeout} s"
        if p.returncode != 0 and not list(d.glob("**/*counter_collection.csv")):
            tail = err.decode(errors="replace").strip().splitlines()[-3:]
            return None, f"rocprofv3 --pmc {counter} exited {p.returncode}: {' | '.join(tail)}"
        dirs[counter] = str(d)
    try:
        res = rocprof_summary.pmc(dirs["FETCH_SIZE"], dirs["WRITE_SIZE"], GEMV_KERNEL, nbytes)
    except SystemExit as e:
        return None, f"counter output incomplete: {e}"
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    res["traffic_over_algorithmic"] = round(res["hbm_bytes_per_launch"] / nbytes, 4)
    return res, None


def tuned_config(N, K, G=128):
    from runtime.model import DecodeConfig, default_gemv_config
    p = pathlib.Path(DecodeConfig().autotune_path)
    best = json.load(open(p)).get("best", {}) if p.exists() else {}
    e = best.get(f"{N}x{K}_G{G}")
    if e is None:
        return default_gemv_config(N, K)
    return tuple(e) if len(e) == 4 else (2, *e)


# Clock-gated timing windows of the standalone kernel legs (runtime.timing.windowed_time): warm_ms of back-to-back
# replays queued ahead of window_ms of timed samples, the shader clock read inside the window. The counter passes
# (traffic_leg) shorten them, since every dispatch under rocprofv3 --pmc is serialized and counted.
WINDOW = {"warm_ms": 300.0, "window_ms": 60.0}


def window_record(w):
    """The timing window's fields that a leg reports."""
    return {"window_samples_us": w["samples_us"], "window_batch": w["batch"], "warm_ms": w["warm_ms"],
            "window_attempts": w["attempts"], "window_clocks": w["clocks"], "throttled": w["throttled"]}


def gemv_leg(Kx, N, Kd, G=128, reps=7):
    """Per-launch duration of the tuned W4A16 GEMV with cold weights: a hipGraph of back-to-back launches over cold
    copies, clock-warmed, `reps` timed samples (runtime.timing.windowed_time); mean_us is the median over the samples
    of the per-launch mean of each."""
    import torch
    from runtime.autotune import gemv_bytes
    from runtime.quant import quantize_pack
    from runtime.timing import ColdCopies, n_copies, windowed_time

    nbytes = gemv_bytes(N, Kd, G)
    g = torch.Generator(device="cuda").manual_seed(N * 7 + Kd)
    packed, sz = quantize_pack((torch.randn(N, Kd, generator=g, device="cuda") * 0.02).half(), G)
    x = torch.randn(Kd, generator=g, device="cuda").half()
    y = torch.empty(N, dtype=torch.half, device="cuda")
    cfg = tuned_config(N, Kd, G)
    cold = ColdCopies([packed, sz], n_copies(nbytes))
    w = windowed_time(lambda i: Kx.gemv_w4a16(*cfg, *cold[i], x, y, G), cold.copies, reps, **WINDOW)
    med = w["median_us"]
    del cold
    return {"N": N, "K": Kd, "group": G, "cfg": list(cfg), "bytes": nbytes, "mean_us": round(med, 3),
            "min_us": round(w["min_us"], 3), "gbps": round(nbytes / med / 1e3, 1),
            "frac": round(nbytes / med / 1e3 / HBM_PEAK_GBS, 4), **window_record(w)}


# read-probe launch shapes swept for the read ceiling: persistent grids of 256..2048 workgroups of 256..1024 threads
# with 4..16 16-byte loads in flight per lane, and the one-load-per-thread full grid (no grid stride) for comparison
PROBE_GRIDS = [(b, t, u) for b in (256, 512, 1024, 2048) for t in (256, 512, 1024) for u in (4, 8, 16)]


def probe_time(Kx, cold, nbytes, blocks, threads, unroll, reps=5, warm_ms=None, window_ms=None):
    import torch
    from runtime.timing import windowed_time
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")      # a one-word sink: the probe writes nothing
    return windowed_time(lambda i: Kx.bw_read(cold[i][0], sink, blocks, threads, unroll), cold.copies, reps,
                         warm_ms=WINDOW["warm_ms"] if warm_ms is None else warm_ms,
                         window_ms=WINDOW["window_ms"] / 2 if window_ms is None else window_ms)


def read_ceiling_leg(Kx, nbytes, reps=5):
    """The read probe over the same byte count, cold, at every launch shape of PROBE_GRIDS plus the full
    one-load-per-thread grid: the best is what a read-only kernel achieves at this size (the GEMV's ceiling)."""
    import torch
    from runtime.timing import ColdCopies, n_copies
    src = torch.empty(nbytes // 16 * 16, dtype=torch.uint8, device="cuda")
    cold = ColdCopies([src], n_copies(nbytes))
    grids = PROBE_GRIDS + [(nbytes // 16 // 512, 512, 1)]
    sweep = []
    for k, (b, t, u) in enumerate(grids):
        w = probe_time(Kx, cold, nbytes, b, t, u, reps, warm_ms=WINDOW["warm_ms"] if k == 0 else 50.0)
        sweep.append({"blocks": b, "threads": t, "unroll": u, "us": round(w["median_us"], 3),
                      "sclk_median": w["clocks"].get("sclk_mhz", {}).get("median"), "throttled": w["throttled"]})
    best = min(sweep, key=lambda r: r["us"])
    full = sweep[-1]
    # the best shape re-timed with the full warm-up and window (the reported figure)
    w = probe_time(Kx, cold, nbytes, best["blocks"], best["threads"], best["unroll"], reps,
                   window_ms=WINDOW["window_ms"])
    del cold
    med = w["median_us"]
    return {"bytes": nbytes, "mean_us": round(med, 3), "gbps": round(nbytes / med / 1e3, 1),
            "frac": round(nbytes / med / 1e3 / HBM_PEAK_GBS, 4),
            "grid": [best["blocks"], best["threads"], best["unroll"]], **window_record(w),
            "full_grid_one_load": {"grid": [full["blocks"], full["threads"], 1], "us": full["us"],
                                   "frac": round(nbytes / full["us"] / 1e3 / HBM_PEAK_GBS, 4)},
            "sweep": sweep}


def read_sweep_leg(Kx, sizes_mb=(2, 4, 8, 16, 31.232, 64, 128, 256, 512), reps=5,
                   grids=((256, 512, 8), (512, 512, 8), (1024, 512, 8), (1024, 1024, 16), (2048, 512, 16))):
    """The read probe over cold copies at sizes from 2 MB to 512 MB (best of a few persistent grids per size), and the
    least-squares fit time = fixed + bytes / bandwidth: the per-launch fixed cost and the streaming bandwidth that
    bound any kernel reading that many bytes once."""
    import torch
    from runtime.timing import ColdCopies, n_copies
    pts = []
    for k, mb in enumerate(sizes_mb):
        nbytes = int(mb * 1e6) // (16 * 512) * (16 * 512)
        cold = ColdCopies([torch.empty(nbytes, dtype=torch.uint8, device="cuda")], n_copies(nbytes, min_copies=2))
        ts = []
        for j, (b, t, u) in enumerate(grids):
            w = probe_time(Kx, cold, nbytes, b, t, u, reps, warm_ms=WINDOW["warm_ms"] if k == j == 0 else 50.0)
            ts.append((w["median_us"], [b, t, u], w["clocks"].get("sclk_mhz", {}).get("median")))
        best = min(ts)
        pts.append({"bytes": nbytes, "us": round(best[0], 3), "grid": best[1], "sclk_median": best[2],
                    "gbps": round(nbytes / best[0] / 1e3, 1), "frac": round(nbytes / best[0] / 1e3 / HBM_PEAK_GBS, 4)})
        del cold
        torch.cuda.empty_cache()
    n = len(pts)
    mx = sum(p["bytes"] for p in pts) / n
    my = sum(p["us"] for p in pts) / n
    slope = sum((p["bytes"] - mx) * (p["us"] - my) for p in pts) / sum((p["bytes"] - mx) ** 2 for p in pts)
    fixed = my - slope * mx
    return {"points": pts, "fit_fixed_us": round(fixed, 3), "fit_gbps": round(1e-3 / slope, 1),
            "fit_frac": round(1e-3 / slope / HBM_PEAK_GBS, 4)}


def calibration_leg(Kx, nbytes, n=16):
    """Known-size kernels for scaling hardware byte counters: n read-probe launches that each read `nbytes` once
    (cold copies) and n device copies of `nbytes` (read + write once). Their FETCH_SIZE / WRITE_SIZE per dispatch,
    divided by nbytes, are the counter-to-HBM-bytes factors (runtime.rocprof_summary)."""
    import torch
    from runtime.timing import ColdCopies
    src = torch.empty(nbytes // 16 * 16, dtype=torch.uint8, device="cuda")
    cold = ColdCopies([src], n + 1)
    sink = torch.zeros(1024 * 8, dtype=torch.int32, device="cuda")
    for i in range(n):
        Kx.bw_read(cold[i][0], sink, 1024, 512, 8)
    torch.cuda.synchronize()
    for i in range(n):
        cold[i + 1][0].copy_(cold[i][0])
    torch.cuda.synchronize()
    del cold


def kernels_leg(Kx, n=64, reps=5):
    """BASELINE configs 2 and 3: the attention ops (32 q / 4 kv heads, D 64, page 16) at contexts 128..4096 and the
    fused elementwise ops at TinyLlama sizes, with GB/s by the algorithmic byte counts: attention 1024 ctx (K and V)
    + 8192 (q, out) + ctx / 4 (block table); add_rmsnorm 10 H; swiglu 6 I; rope_append 4 D (n_q + 2 n_kv). Part size
    and kernel choice are the runtime's attention policy for each context; the reference op gets the policy's part
    size (its caller passes it, runtime/model.py:160-178 of the reference) and version 3.
    Attention is timed cold, as the reference times it with its read flush between iterations
    (bench/kernel_bench.py:147-160, bench/timing.py:28-32): a clock-warmed hipGraph of back-to-back launches, each on
    its own copy of the paged K/V, the copies together well over the 256 MB MALL (keys *_us, *_gbps); the hot figure
    (one K/V for n launches, L2-resident) is kept beside it (*_hot_us). The elementwise ops are timed hot (their
    operands are 10-34 KB; in the decode step they come from the producing kernel through L2)."""
    import math
    import torch
    from runtime.model import DecodeConfig, rope_tables
    from runtime.timing import ColdCopies, graph_time, n_copies, windowed_time

    dev = "cuda"
    pol = [e for e in json.load(open(DecodeConfig().attn_policy_path)).get("policy", []) if e["max_ctx"] < (1 << 30)]

    def entry(ctx):
        below = [e for e in pol if e["max_ctx"] <= ctx]
        return below[-1] if below else (pol[0] if pol else {"part_size": 64, "impl": 1})

    n_q, n_kv, D, P = 32, 4, 64, 16
    out = {"attention": {}, "fused": {}}
    for ctx in (128, 512, 2048, 4096):
        g = torch.Generator(device=dev).manual_seed(ctx)
        pages = ctx // P + 3
        kc = torch.randn(pages, n_kv, P, D, generator=g, device=dev).half()
        vc = torch.randn(pages, n_kv, P, D, generator=g, device=dev).half()
        bt = torch.randperm(pages, generator=g, device=dev).int()
        q = torch.randn(n_q * D, generator=g, device=dev).half()
        qkv = torch.randn((n_q + 2 * n_kv) * D, generator=g, device=dev).half()
        pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
        cos, sin = (t.to(dev) for t in rope_tables(ctx + 1, D))
        e = entry(ctx)
        ps, impl = e["part_size"], e.get("impl", 1)
        S = math.ceil(ctx / ps)
        f32 = dict(dtype=torch.float32, device=dev)
        o_part, m_part, l_part = torch.empty(n_q, S, D, **f32), torch.empty(n_q, S, **f32), torch.empty(n_q, S, **f32)
        o = torch.empty(n_q, D, dtype=torch.half, device=dev)
        nbytes = 1024 * ctx + 8192 + ctx // 4
        hot_ref = graph_time(lambda i: Kx.paged_attention(q, kc, vc, bt, pos, ps, o_part, m_part, l_part, o, 3), n,
                             reps)[1]
        hot_dec = graph_time(lambda i: Kx.attention_decode(qkv, cos, sin, pos, bt, kc, vc, n_q, n_kv, ps, o_part,
                                                           m_part, l_part, o, impl), n, reps)[1]
        kv = ColdCopies([kc, vc], n_copies(2 * kc.numel() * 2))
        w_ref = windowed_time(lambda i: Kx.paged_attention(q, *kv[i], bt, pos, ps, o_part, m_part, l_part, o, 3),
                              kv.copies, reps, warm_ms=100.0, window_ms=30.0)
        w_dec = windowed_time(lambda i: Kx.attention_decode(qkv, cos, sin, pos, bt, *kv[i], n_q, n_kv, ps, o_part,
                                                            m_part, l_part, o, impl),
                              kv.copies, reps, warm_ms=30.0, window_ms=30.0)
        del kv
        t_ref, t_dec = w_ref["median_us"], w_dec["median_us"]
        out["attention"][str(ctx)] = {
            "bytes": nbytes, "part_size": ps, "paged_attention_v3_us": round(t_ref, 3),
            "paged_attention_v3_gbps": round(nbytes / t_ref / 1e3, 1), "paged_attention_v3_hot_us": round(hot_ref, 3),
            "attention_decode_impl": impl, "attention_decode_us": round(t_dec, 3),
            "attention_decode_gbps": round(nbytes / t_dec / 1e3, 1), "attention_decode_hot_us": round(hot_dec, 3),
            "ref_over_decode": round(t_ref / t_dec, 4),
            "sclk_median": w_ref["clocks"].get("sclk_mhz", {}).get("median"),
            "throttled": bool(w_ref["throttled"] or w_dec["throttled"])}
    g = torch.Generator(device=dev).manual_seed(3)
    H, I = 2048, 5632
    x = torch.randn(H, generator=g, device=dev).half()
    zero = torch.zeros(H, dtype=torch.half, device=dev)
    w = torch.randn(H, generator=g, device=dev).half()
    normed = torch.empty(H, dtype=torch.half, device=dev)
    gu = torch.randn(2 * I, generator=g, device=dev).half()
    act = torch.empty(I, dtype=torch.half, device=dev)
    pages = 512 // P + 3
    kc = torch.zeros(pages, n_kv, P, D, dtype=torch.half, device=dev)
    vc = torch.zeros_like(kc)
    bt = torch.arange(pages, dtype=torch.int32, device=dev)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=g, device=dev).half()
    cos, sin = (t.to(dev) for t in rope_tables(513, D))
    pos = torch.tensor([511], dtype=torch.int32, device=dev)
    for name, nbytes, fn in (
            ("add_rmsnorm_2048", 10 * H, lambda i: Kx.add_rmsnorm(x, zero, w, normed, 1e-5)),
            ("swiglu_5632", 6 * I, lambda i: Kx.swiglu(gu, act)),
            ("rope_append_32q4kv_d64", 4 * D * (n_q + 2 * n_kv),
             lambda i: Kx.rope_append(qkv, cos, sin, pos, bt, kc, vc, n_q, n_kv))):
        w = windowed_time(fn, n, reps, warm_ms=30.0, window_ms=20.0)
        t = w["median_us"]
        out["fused"][name] = {"bytes": nbytes, "us": round(t, 3), "gbps": round(nbytes / t / 1e3, 2),
                              "frac": round(nbytes / t / 1e3 / HBM_PEAK_GBS, 5),
                              "sclk_median": w["clocks"].get("sclk_mhz", {}).get("median")}
    return out


def attn8b_leg(Kx, ctx=4096, reps=5, eager=8, part_size=0):
    """Decode attention of BASELINE config 5 alone: Llama-3-8B heads (32 q / 8 kv, D 128, page 16) at context ctx,
    the reference op (split kernel + combine) with the runtime's policy entry for that context, each launch on a
    different cold copy of the paged K/V (block table a seeded permutation), then the read probe over the same K/V
    bytes on the split kernel's workgroup count and on a whole-chip persistent grid. Timed as clock-warmed hipGraphs
    of back-to-back launches (runtime.timing.windowed_time); `eager`
    extra launches of each run outside any graph first, for the counter passes (rocprofv3 --pmc over this leg).
    part_size > 0 replaces the policy's split size (lean kernel when it fits, else the block kernel)."""
    import math
    import torch
    from runtime.model import DecodeConfig, Model
    from runtime.timing import ColdCopies, n_copies, windowed_time

    dev = "cuda"
    n_q, n_kv, D, P = 32, 8, 128, 16
    cap = ctx + 48
    ent = Model._policy_entry_of(json.load(open(DecodeConfig().attn_policy_path)), D, cap)
    ps, impl = ent["part_size"], ent.get("impl", 1)
    if part_size > 0:
        ps, impl = part_size, (3 if part_size % 16 == 0 and part_size <= 256 else 1)
    version = 5 if impl == 3 else 3
    S = math.ceil(cap / ps)
    pages = math.ceil(cap / P)
    g = torch.Generator(device=dev).manual_seed(ctx)
    kc = torch.randn(pages, n_kv, P, D, generator=g, device=dev).half()
    vc = torch.randn(pages, n_kv, P, D, generator=g, device=dev).half()
    kv = ColdCopies([kc, vc], n_copies(2 * kc.numel() * 2))
    del kc, vc
    bt = torch.randperm(pages, generator=g, device=dev).int()
    q = torch.randn(n_q * D, generator=g, device=dev).half()
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    o_part, m_part, l_part = torch.empty(n_q, S, D, **f32), torch.empty(n_q, S, **f32), torch.empty(n_q, S, **f32)
    o = torch.empty(n_q, D, dtype=torch.half, device=dev)
    kv_bytes = 2 * ctx * n_kv * D * 2
    nbytes = kv_bytes + 2 * n_q * D * 2 + 4 * math.ceil(ctx / P)
    attn = lambda i: Kx.paged_attention(q, *kv[i], bt, pos, ps, o_part, m_part, l_part, o, version)
    src = ColdCopies([torch.empty(kv_bytes, dtype=torch.uint8, device=dev)], n_copies(kv_bytes))
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    grids = {"split_workgroups": (n_kv * S, 512, 8), "whole_chip": (1024, 512, 8)}
    reads = {k: (lambda i, b=b: Kx.bw_read(src[i][0], sink, *b)) for k, b in grids.items()}
    for i in range(eager):
        attn(i)
    for fn in reads.values():
        for i in range(eager):
            fn(i)
    torch.cuda.synchronize()
    w = windowed_time(attn, kv.copies, reps, warm_ms=200.0, window_ms=30.0)
    t_attn = w["median_us"]
    res = {"ctx": ctx, "part_size": ps, "splits": S, "version": version, "bytes": nbytes,
           "us": round(t_attn, 3), "gbps": round(nbytes / t_attn / 1e3, 1),
           "frac": round(nbytes / t_attn / 1e3 / HBM_PEAK_GBS, 4),
           "sclk_median": w["clocks"].get("sclk_mhz", {}).get("median"), "throttled": w["throttled"], "bw_read": {}}
    for k, fn in reads.items():
        t = windowed_time(fn, src.copies, reps, warm_ms=50.0, window_ms=30.0)["median_us"]
        res["bw_read"][k] = {"grid": list(grids[k]), "bytes": kv_bytes, "us": round(t, 3),
                             "gbps": round(kv_bytes / t / 1e3, 1)}
    del kv, src
    return res


def decode_leg(model, ctx, steps, warmup):
    """`steps` decode steps from context ctx after `warmup` untimed ones. The throughput comes from one pass with HIP
    events only at its two ends; the per-token distribution (median, quartiles: bench/e2e.py:178-197) from a second
    pass over the same positions with an event pair around every step, because those events cost the stream about
    10 us per TinyLlama step (495-498 against 485-486 us per step, same model and box)."""
    import torch
    model.reset(ctx)
    for _ in range(warmup):
        model.run_step()
    torch.cuda.synchronize()
    model.reset(ctx)
    from runtime.timing import clock_summary, gpu_sysfs_dir, read_clocks
    pci = gpu_sysfs_dir()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        model.run_step()
    end.record()
    samples = []                                   # clocks read while the timed steps run
    while not end.query():
        if start.query():
            c = read_clocks(pci)
            if c:
                samples.append(c)
        time.sleep(0.0005)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(end)
    model.reset(ctx)
    per = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for s, e in per:
        s.record()
        model.run_step()
        e.record()
    torch.cuda.synchronize()
    tok_us = sorted(s.elapsed_time(e) * 1e3 for s, e in per)
    return {"ctx_start": ctx, "steps": steps, "ms_per_step": total_ms / steps, "tok_s": steps / (total_ms / 1e3),
            "median_us": statistics.median(tok_us), "p10_us": tok_us[len(tok_us) // 10],
            "p90_us": tok_us[(9 * len(tok_us)) // 10], **token_quartiles(tok_us), "wall_tok_s": steps / wall,
            "window_clocks": clock_summary(samples)}


def decode_8b_leg(ctx=4096, steps=64, warmup=8):
    """Llama-3-8B-architecture W4A16 decode at context `ctx`, hipGraph replay, once with the INT4
    LM head and once with the fp16 one (the config leaves the head format open)."""
    import torch
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LLAMA3_8B, SyntheticLlama

    out = {}
    for head in ("int4", "fp16"):
        t0 = time.perf_counter()
        m = Model(SyntheticLlama(LLAMA3_8B, seed=0), LLAMA3_8B,
                  DecodeConfig(lm_head=head, max_ctx=ctx + steps + warmup + 16))
        m.prepare(ctx + steps + warmup + 16)
        built = time.perf_counter() - t0
        d = decode_leg(m, ctx, steps, warmup)
        bpt = m.bytes_per_token(ctx + steps // 2)
        roof = HBM_PEAK_GBS * 1e9 / bpt
        out[f"{head}_head"] = {"tok_s": round(d["tok_s"], 2), "median_us": round(d["median_us"], 2),
                               "bytes_per_token": bpt, "roofline_tok_s": round(roof, 1),
                               "frac_of_roofline": round(d["tok_s"] / roof, 4), "part_size": m.part_size,
                               "build_s": round(built, 1)}
        log(f"llama3-8b ctx {ctx} {head} head: {d['tok_s']:.1f} tok/s, median {d['median_us']:.1f} us "
            f"({d['tok_s'] / roof:.1%} of the {roof:.0f} tok/s roofline)")
        if head == "int4":
            out["prefill_512"] = prefill_leg(m, reps=3)
            log(f"llama3-8b prefill 512: {out['prefill_512']['ms']:.2f} ms ({out['prefill_512']['tflops']:.0f} TFLOP/s)")
        del m
        torch.cuda.empty_cache()
    return out


def prefill_leg(model, M=512, reps=5):
    """Prompt processing: model.prefill of an M-token prompt from position 0 (W4A16 GEMMs, batched rope/append and
    norms, causal prefill attention), against teacher-forcing the same prompt through the decode step's hipGraph.
    The compute roofline is 2 x (projection weights) x M FLOPs plus the attention's 4 x n_q x D x (sum of contexts)
    at MI355X's dense fp16 MFMA peak."""
    import torch
    prompt = torch.randint(0, model.V, (M,), generator=torch.Generator().manual_seed(7))
    times = []
    for _ in range(reps + 1):
        model.reset(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.prefill(prompt)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    pf = statistics.median(times[1:])
    model.reset(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.teacher_force(prompt)
    torch.cuda.synchronize()
    tf = time.perf_counter() - t0
    gemms = {}
    lw = model.layers[0]
    for key, epi in (("qkv", 0), ("o", 0), ("gu", 1), ("down", 0)):
        lin = lw[key]
        if not lin.quant:
            continue
        gemms[f"{key}_{lin.N}x{lin.K}"] = gemm_timing(model, lin, M, epi)
    params = sum(l[k].N * l[k].K for l in model.layers for k in ("qkv", "o", "gu", "down"))
    flops = 2 * params * M + model.L * 4 * model.n_q * model.D * (M * (M + 1) // 2)
    return {"prompt_tokens": M, "ms": round(pf * 1e3, 3), "tok_s": round(M / pf, 1),
            "tflops": round(flops / pf / 1e12, 1), "frac_of_fp16_mfma_peak": round(flops / pf / 2.5e15, 4),
            "teacher_force_ms": round(tf * 1e3, 2), "speedup_vs_teacher_force": round(tf / pf, 1), "gemm": gemms}


def gemm_timing(model, lin, M, epilogue, reps=20):
    """One prefill projection on its own: dk_gemm_w4a16 (the model's packed weights, SwiGLU epilogue for gate|up) and,
    for comparison, hipBLASLt's fp16 GEMM (torch.mm) on fp16 weights of the same shape; HIP events, mean of reps."""
    import torch
    dev = model.cfg.device
    x = torch.randn(M, lin.K, generator=torch.Generator().manual_seed(3)).half().to(dev)
    y = torch.empty(M, lin.N // (1 + epilogue), dtype=torch.half, device=dev)

    def timed(fn):
        for _ in range(3):
            fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / reps

    us = timed(lambda: model.gemm(lin, x, y, epilogue))
    w16 = torch.randn(lin.N, lin.K, device=dev).half()
    yb = torch.empty(M, lin.N, dtype=torch.half, device=dev)
    ub = timed(lambda: torch.mm(x, w16.t(), out=yb))
    fl = 2 * M * lin.N * lin.K
    return {"us": round(us, 2), "tflops": round(fl / us / 1e6, 1), "hipblaslt_fp16_us": round(ub, 2),
            "hipblaslt_fp16_tflops": round(fl / ub / 1e6, 1)}


GEMM_SHAPES = (("llama3_8b.gate_up", 28672, 4096, 1), ("llama3_8b.qkv", 6144, 4096, 0), ("llama3_8b.o", 4096, 4096, 0),
               ("llama3_8b.down", 4096, 14336, 0), ("tinyllama.gate_up", 11264, 2048, 1),
               ("tinyllama.qkv", 2560, 2048, 0), ("tinyllama.down", 2048, 5632, 0))


def gemm_leg(Kx, M=512, reps=5, eager=4, G=128):
    """The prefill projections alone: dk_gemm_w4a16 at M prompt rows over the Llama-3-8B and TinyLlama shapes (SwiGLU
    epilogue for gate|up), clock-warmed graph windows, beside hipBLASLt's fp16 GEMM (torch.mm) on fp16 weights of the
    same shape; `eager` extra launches of each run outside any graph first, for the counter passes (rocprofv3 --pmc
    over this leg)."""
    import torch
    from runtime.quant import quantize_pack
    from runtime.timing import windowed_time
    out = {}
    g = torch.Generator(device="cuda").manual_seed(11)
    for name, N, K, epi in GEMM_SHAPES:
        packed, sz = quantize_pack((torch.randn(N, K, generator=g, device="cuda") * 0.02).half(), G)
        x = torch.randn(M, K, generator=g, device="cuda").half()
        y = torch.empty(M, N // (1 + epi), dtype=torch.half, device="cuda")
        wsb = Kx.gemm_workspace_bytes(M, N, K, G, epi)     # split-K workspace, as Model.gemm passes it
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda") if wsb else None
        for _ in range(eager):
            Kx.gemm_w4a16(packed, sz, x, y, G, epilogue=epi, workspace=ws)
        torch.cuda.synchronize()
        w = windowed_time(lambda i: Kx.gemm_w4a16(packed, sz, x, y, G, epilogue=epi, workspace=ws), 8, reps,
                          warm_ms=100.0, window_ms=40.0)
        w16 = torch.randn(N, K, generator=g, device="cuda").half()
        yb = torch.empty(M, N, dtype=torch.half, device="cuda")
        wb = windowed_time(lambda i: torch.mm(x, w16.t(), out=yb), 8, reps, warm_ms=30.0, window_ms=40.0)
        fl = 2 * M * N * K
        out[name] = {"M": M, "N": N, "K": K, "epilogue": epi, "splitk_workspace_bytes": wsb, "us": round(w["median_us"], 2),
                     "tflops": round(fl / w["median_us"] / 1e6, 1), "hipblaslt_fp16_us": round(wb["median_us"], 2),
                     "hipblaslt_fp16_tflops": round(fl / wb["median_us"] / 1e6, 1),
                     "sclk_median": w["clocks"].get("sclk_mhz", {}).get("median")}
        log(f"gemm {name} {M}x{N}x{K}: {out[name]['us']} us ({out[name]['tflops']} TFLOP/s), hipBLASLt fp16 "
            f"{out[name]['hipblaslt_fp16_us']} us")
        del packed, sz, w16, yb, ws
        torch.cuda.empty_cache()
    return out


def token_quartiles(tok_us):
    """First and third quartile and the interquartile range of per-token times in us (bench/timing.py:134-138 of the
    reference reports median + IQR); empty for fewer than two tokens."""
    if len(tok_us) < 2:
        return {}
    q = statistics.quantiles(sorted(tok_us), n=4, method="inclusive")
    return {"q1_us": q[0], "q3_us": q[2], "iqr_us": q[2] - q[0]}


def step_stats(times_s):
    """Median and interquartile range of per-step times (the reference's statistics, bench/timing.py:134-138)."""
    t = sorted(times_s)
    q = statistics.quantiles(t, n=4, method="inclusive")
    return {"n": len(t), "median_ms": round(statistics.median(t) * 1e3, 2), "q1_ms": round(q[0] * 1e3, 2),
            "q3_ms": round(q[2] * 1e3, 2), "iqr_ms": round((q[2] - q[0]) * 1e3, 2)}


def cpu_baseline_leg(model, shape, ctxs=(512, CTX_LONG), warmup=5, steps=30):
    """The CPU oracle's decode step on the host cores: `warmup` untimed then `steps` timed steps at each context
    (positions ctx, ctx + 1, ...; the cache below ctx holds zeros, which costs the same as real keys), timed one step
    at a time with perf_counter. value = 1 / median step time at the first context."""
    import torch
    from __graft_entry__ import _ref_weights
    from oracle.decode_ref import RefDecoder

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    weights = _ref_weights(model, shape)
    prep = time.perf_counter() - t0
    per_ctx = {}
    for ctx in ctxs:
        cap = ctx + warmup + steps + 2
        dec = RefDecoder(weights, shape, max_ctx=cap, page=model.cfg.page,
                         block_table=torch.arange(cap // model.cfg.page + 2, dtype=torch.int32))
        times = []
        for i in range(warmup + steps):
            s = time.perf_counter()
            dec.step(1 + i, ctx + i)
            times.append(time.perf_counter() - s)
        st = step_stats(times[warmup:])
        st["tok_s"] = round(1e3 / st["median_ms"], 3)
        per_ctx[str(ctx)] = st
        log(f"cpu baseline ctx {ctx}: median {st['median_ms']} ms/token (IQR {st['iqr_ms']} ms) on {cores} cores")
    first = per_ctx[str(ctxs[0])]
    return {"value": first["tok_s"], "unit": "tok/s", "cores": cores, "kind": "port", "per_ctx": per_ctx,
            "sample": f"TinyLlama decode steps of oracle.decode_ref (torch fp32 CPU restatement of the reference "
                      f"backend='ref' composition, runtime/model.py:216-233) on the same dequantized weights: "
                      f"{warmup} warm-up + {steps} timed steps at each of ctx {', '.join(map(str, ctxs))}; value = "
                      f"1 / median step at ctx {ctxs[0]}; weights dequantized on the CPU once ({prep:.1f} s, "
                      f"untimed)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--leg", choices=("all", "gemv", "kernels", "decode", "decode8b", "attn8b", "readsweep",
                                      "readceiling", "prefill", "gemm"),
                    default="all",
                    help="gemv: the 4096x14336 GEMV and its calibration copies only; decode: the TinyLlama decode "
                         "step only; decode8b: the Llama-3-8B decode legs only; attn8b: the Llama-3-8B ctx-4096 "
                         "attention alone and the read probe over its K/V bytes; readsweep: the read probe from 2 "
                         "to 512 MB and its fixed-cost + bandwidth fit; readceiling: the read probe's launch-shape "
                         "sweep at the roofline GEMV's byte count; gemm: the prefill GEMM alone at the Llama-3-8B and "
                         "TinyLlama projection shapes, M 512, beside hipBLASLt fp16; prefill: the TinyLlama prefill leg only; "
                         "kernels: the attention and fused-op kernels of configs 2 and 3 only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--attn-part", type=int, default=0, help="attn8b: split size instead of the policy's")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes")
    ap.add_argument("--warm-ms", type=float, default=WINDOW["warm_ms"],
                    help="GPU time of back-to-back replays ahead of each standalone kernel's timed window")
    ap.add_argument("--window-ms", type=float, default=WINDOW["window_ms"],
                    help="GPU time of a standalone kernel's timed samples")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only: the batch-1 decode path is single-GPU by design and every box here "
              f"has one GPU (got --gpus {a.gpus}). Across GPUs the path would shard by tensor parallelism: qkv and "
              f"gate|up column-parallel, o and down row-parallel with one all-reduce each, attention by kv head",
              file=sys.stderr)
        sys.exit(2)

    from runtime.autotune import gemv_bytes

    WINDOW.update({"warm_ms": a.warm_ms, "window_ms": a.window_ms})
    # the counter passes run in child processes before this process touches the GPU
    traffic, traffic_note = None, "not measured (--no-traffic)"
    if a.leg == "all" and not a.no_traffic:
        traffic, traffic_note = traffic_leg(gemv_bytes(4096, 14336, 128))
        log(f"traffic: {traffic['hbm_bytes_per_launch'] if traffic else None} B per launch "
            f"({traffic['traffic_over_algorithmic'] if traffic else traffic_note})")

    import torch
    from runtime import ext

    Kx = ext.load()
    dev_name = torch.cuda.get_device_properties(0).name
    if a.leg == "gemv":
        g1 = gemv_leg(Kx, 4096, 14336)
        log(f"gemv 4096x14336 {g1['cfg']}: {g1['mean_us']:.3f} us/launch -> {g1['gbps']:.0f} GB/s ({g1['frac']:.1%})")
        calibration_leg(Kx, g1["bytes"])
        print(json.dumps({"leg": "gemv", "gemv_4096x14336": g1}), flush=True)
        return

    if a.leg == "kernels":
        print(json.dumps({"leg": "kernels", "kernels_cfg2_cfg3": kernels_leg(Kx)}), flush=True)
        return

    if a.leg == "decode8b":
        print(json.dumps({"leg": "decode8b", "decode_llama3_8b_ctx4096": decode_8b_leg()}), flush=True)
        return

    if a.leg == "readsweep":
        r = read_sweep_leg(Kx)
        log(f"read probe: time = {r['fit_fixed_us']} us + bytes / {r['fit_gbps']} GB/s; " +
            ", ".join(f"{p['bytes'] / 1e6:.0f} MB {p['us']} us ({p['frac']:.0%})" for p in r["points"]))
        print(json.dumps({"leg": "readsweep", "read_sweep": r}), flush=True)
        return

    if a.leg == "gemm":
        print(json.dumps({"leg": "gemm", "gemm_512": gemm_leg(Kx)}), flush=True)
        return

    if a.leg == "readceiling":
        rc = read_ceiling_leg(Kx, gemv_bytes(4096, 14336, 128))
        log(f"read probe of {rc['bytes']} B: best {rc['grid']} {rc['mean_us']:.3f} us -> {rc['gbps']:.0f} GB/s "
            f"({rc['frac']:.1%}); one load per thread over the full grid {rc['full_grid_one_load']['us']} us")
        print(json.dumps({"leg": "readceiling", "read_ceiling": rc}), flush=True)
        return

    if a.leg == "attn8b":
        r = attn8b_leg(Kx, part_size=a.attn_part)
        log(f"llama3-8b attention ctx {r['ctx']} (part {r['part_size']}, {r['splits']} splits): {r['us']:.3f} us -> "
            f"{r['gbps']:.0f} GB/s; read probe over the K/V bytes: " +
            ", ".join(f"{k} {v['us']:.3f} us" for k, v in r["bw_read"].items()))
        print(json.dumps({"leg": "attn8b", "attention_llama3_8b_ctx4096": r}), flush=True)
        return

    from runtime.model import DecodeConfig, Model
    from runtime.synth import TINYLLAMA, SyntheticLlama

    clocks = {}

    def sampled(name, fn, *args, **kw):
        with ClockSampler() as cs:
            r = fn(*args, **kw)
        clocks[name] = cs.summary()
        return r

    # the standalone GEMV and kernel legs first, while no model occupies the device (cold weights either way); the
    # decode and prefill legs alone skip them, so that their kernel traces hold only the model's kernels
    if a.leg == "all":
        g1 = sampled("gemv_4096x14336", gemv_leg, Kx, 4096, 14336)
        log(f"gemv 4096x14336 {g1['cfg']}: {g1['mean_us']:.3f} us/launch -> {g1['gbps']:.0f} GB/s ({g1['frac']:.1%})")
        g2 = sampled("gemv_14336x4096", gemv_leg, Kx, 14336, 4096)
        log(f"gemv 14336x4096 {g2['cfg']}: {g2['mean_us']:.3f} us/launch -> {g2['gbps']:.0f} GB/s ({g2['frac']:.1%})")
        g3 = sampled("gemv_5632x2048", gemv_leg, Kx, 5632, 2048)
        log(f"gemv 5632x2048 {g3['cfg']}: {g3['mean_us']:.3f} us/launch -> {g3['gbps']:.0f} GB/s ({g3['frac']:.1%})")
        rc = sampled("read_ceiling", read_ceiling_leg, Kx, g1["bytes"])
        log(f"read probe of {rc['bytes']} B: best {rc['grid']} {rc['mean_us']:.3f} us -> {rc['gbps']:.0f} GB/s "
            f"({rc['frac']:.1%})")
        kern = sampled("kernels", kernels_leg, Kx)
        log("attention (cfg2) us: " + ", ".join(f"ctx {c}: ref op {v['paged_attention_v3_us']}, fused "
                                              f"{v['attention_decode_us']}" for c, v in kern["attention"].items()))
        log("fused ops (cfg3) us: " + ", ".join(f"{k} {v['us']}" for k, v in kern["fused"].items()))

    caps = leg_caps(a.ctx, a.steps, a.warmup)
    log(f"device {dev_name}; building TinyLlama-shape W4A16 model (max_ctx {caps['max_ctx']})")
    t0 = time.perf_counter()
    model = Model(SyntheticLlama(TINYLLAMA, seed=0), TINYLLAMA, DecodeConfig(lm_head="fp16", max_ctx=caps["max_ctx"]))
    model.prepare(caps["decode"])
    log(f"model built + graph captured in {time.perf_counter() - t0:.1f}s (part_size {model.part_size}, "
        f"max_splits {model.max_splits})")
    dec = sampled("decode", decode_leg, model, a.ctx, a.steps, a.warmup)
    log(f"decode ctx {a.ctx}: {dec['tok_s']:.1f} tok/s, median {dec['median_us']:.1f} us/token")
    if a.leg == "decode":
        print(json.dumps({"leg": "decode", "decode": dec, "clocks": clocks}), flush=True)
        return
    if a.leg == "prefill":
        model.prepare(caps["prefill"])
        print(json.dumps({"leg": "prefill", "prefill_tinyllama_512": prefill_leg(model, PREFILL_TOKENS)}), flush=True)
        return
    bpt = model.bytes_per_token(a.ctx + a.steps // 2)
    model.prepare(caps["decode_long"])
    dec2k = sampled("decode_ctx2048", decode_leg, model, CTX_LONG, CTX_LONG_STEPS, CTX_LONG_WARMUP)
    log(f"decode ctx {CTX_LONG}: {dec2k['tok_s']:.1f} tok/s")
    bpt2k = model.bytes_per_token(CTX_LONG + CTX_LONG_STEPS // 2)

    model.prepare(caps["prefill"])
    pre = sampled("prefill", prefill_leg, model, PREFILL_TOKENS)
    log(f"prefill {pre['prompt_tokens']} tokens: {pre['ms']:.2f} ms ({pre['tok_s']:.0f} tok/s, {pre['tflops']:.0f} "
        f"TFLOP/s, {pre['speedup_vs_teacher_force']:.0f}x teacher forcing)")

    d8b = sampled("decode_llama3_8b", decode_8b_leg)

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline_leg(model, TINYLLAMA)
        log(f"cpu baseline: {cpu['value']:.3f} tok/s on {cpu['cores']} cores")

    out = {
        "metric": METRIC, "value": round(dec["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(dec["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "w4a16 (int4 weights, fp16 activations, fp32 accumulate)",
        "data": "synthetic (random-init weights N(0,0.02), random token ids)",
        "config": {"workload": "TinyLlama-1.1B-architecture W4A16 G128 decode step (BASELINE config 4), fp16 LM head, "
                               "hipGraph replay, batch 1", "context_start": a.ctx, "global_batch": 1,
                   "parallelism": "single GPU", "device": dev_name},
        "roofline": {"bound": "hbm", "kernel": f"gemv_w4a16 4096x14336 G128 cfg {g1['cfg']}",
                     "achieved": g1["gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": g1["frac"],
                     "traffic": traffic["hbm_bytes_per_launch"] if traffic else None,
                     "traffic_detail": traffic or traffic_note, "bytes_per_launch": g1["bytes"],
                     "mean_us": g1["mean_us"], "read_ceiling_frac": rc["frac"],
                     "frac_of_read_ceiling": round(rc["mean_us"] / g1["mean_us"], 4),
                     "window_sclk_mhz": g1["window_clocks"].get("sclk_mhz"), "throttled": g1["throttled"]},
        "gemv_4096x14336": g1, "gemv_14336x4096": g2, "gemv_cfg1_5632x2048": g3, "read_ceiling": rc,
        "kernels_cfg2_cfg3": kern,
        "decode": {**{k: round(v, 3) if isinstance(v, float) else v for k, v in dec.items()},
                   "bytes_per_token": bpt, "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
                   "frac_of_roofline": round(dec["tok_s"] / (HBM_PEAK_GBS * 1e9 / bpt), 4)},
        "decode_ctx2048": {"tok_s": round(dec2k["tok_s"], 2), "median_us": round(dec2k["median_us"], 2),
                           "p10_us": round(dec2k["p10_us"], 2), "p90_us": round(dec2k["p90_us"], 2),
                           "iqr_us": round(dec2k["iqr_us"], 2),
                           "bytes_per_token": bpt2k,
                           "frac_of_roofline": round(dec2k["tok_s"] / (HBM_PEAK_GBS * 1e9 / bpt2k), 4)},
        "prefill_tinyllama_512": pre,
        "decode_llama3_8b_ctx4096": d8b,
        "clocks": clocks,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
