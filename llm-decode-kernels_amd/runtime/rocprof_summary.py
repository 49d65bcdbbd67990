"""Summaries of rocprofv3 CSV output (``--output-format csv``) for the measurements reported by bench.py.

    python -m runtime.rocprof_summary stats <rocprof dir> [--top 20]
        per-kernel calls / average / min / max duration and share of GPU time, from *_kernel_stats.csv

    python -m runtime.rocprof_summary pmc --fetch <dir> --write <dir> --kernel <substring> --bytes <B> [--out f.json]
        HBM bytes per dispatch of the kernel whose name contains <substring>, from one FETCH_SIZE pass and one
        WRITE_SIZE pass over ``bench.py --leg gemv``. The counters are scaled by what they read for kernels of known
        size run in the same process (bench.py calibration_leg): the read probe streaming B bytes once (FETCH_SIZE per B read)
        and the last 16 device copies of B bytes (WRITE_SIZE per B written).

    python -m runtime.rocprof_summary counters <dir> [<dir> ...] [--kernel <substring> ...] [--out f.json]
        Per kernel launch shape (name, grid, workgroup): the mean per dispatch of every counter found in the
        counter_collection.csv files of the given passes, and the ratios derived from them when their counters are
        present: mean L2 read latency seen by the vector caches (TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ, cycles),
        mean HBM-side read latency (TCC_EA0_RDREQ_LEVEL / TCC_EA0_RDREQ, Little's law, cycles), the share of wave
        time spent waiting on a memory dependency (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES), vector reads per wave, and
        the L2 hit rate.
"""
import argparse
import csv
import glob
import json
import os
import statistics
import sys


def _one(pattern):
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise SystemExit(f"no file matches {pattern}")
    return hits[0]


def _short(name, n=72):
    for pre in ("_ZN2dk12_GLOBAL__N_1", "void dk::(anonymous namespace)::"):
        if name.startswith(pre):
            name = name[len(pre):]
    return name if len(name) <= n else name[: n - 3] + "..."


def stats(d, top=20):
    rows = list(csv.DictReader(open(_one(os.path.join(d, "**", "*kernel_stats.csv")))))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    lines = [f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'share':>6}  kernel"]
    for r in rows[:top]:
        lines.append(f"{int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.3f} {float(r['MinNs']) / 1e3:9.3f} "
                     f"{float(r['MaxNs']) / 1e3:9.3f} {100 * float(r['TotalDurationNs']) / total:5.1f}%  "
                     f"{_short(r['Name'])}")
    return "\n".join(lines)


def _counter_rows(d, counter):
    f = _one(os.path.join(d, "**", "*counter_collection.csv"))
    rows = [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def pmc(fetch_dir, write_dir, kernel, nbytes, n_cal=16):
    fr = _counter_rows(fetch_dir, "FETCH_SIZE")
    wr = _counter_rows(write_dir, "WRITE_SIZE")
    kib = lambda rs: [float(r["Counter_Value"]) * 1024 for r in rs]
    g_f = kib([r for r in fr if kernel in r["Kernel_Name"]])
    g_w = kib([r for r in wr if kernel in r["Kernel_Name"]])
    rd = kib([r for r in fr if "read_probe_kernel" in r["Kernel_Name"]][-n_cal:])
    cp = kib([r for r in wr if "copyBuffer" in r["Kernel_Name"]][-n_cal:])
    if not (g_f and g_w and rd and cp):
        raise SystemExit("missing dispatches: need the kernel, read-probe and copy dispatches in both passes")
    f_factor = statistics.median(rd) / nbytes
    w_factor = statistics.median(cp) / nbytes
    fetch = statistics.mean(g_f) / f_factor
    write = statistics.mean(g_w) / w_factor
    return {"kernel": kernel, "dispatches": len(g_f), "fetch_size_kib_per_dispatch": round(statistics.mean(g_f) / 1024, 3),
            "write_size_kib_per_dispatch": round(statistics.mean(g_w) / 1024, 3),
            "fetch_factor": round(f_factor, 5), "write_factor": round(w_factor, 5),
            "hbm_read_bytes_per_launch": round(fetch), "hbm_write_bytes_per_launch": round(write),
            "hbm_bytes_per_launch": round(fetch + write)}


def _derive(c):
    d = {}
    ratio = lambda a, b: round(c[a] / c[b], 4) if a in c and c.get(b) else None
    for key, a, b in (("l2_read_latency_cycles", "TCP_TCC_READ_REQ_LATENCY_sum", "TCP_TCC_READ_REQ_sum"),
                      ("hbm_read_latency_cycles", "TCC_EA0_RDREQ_LEVEL_sum", "TCC_EA0_RDREQ_sum"),
                      ("wave_time_waiting_on_memory", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES"),
                      ("wave_time_waiting_any", "SQ_WAIT_ANY", "SQ_WAVE_CYCLES"),
                      ("vmem_reads_per_wave", "SQ_INSTS_VMEM_RD", "SQ_WAVES"),
                      ("l2_read_requests_per_wave", "TCP_TCC_READ_REQ_sum", "SQ_WAVES"),
                      ("hbm_read_requests_per_wave", "TCC_EA0_RDREQ_sum", "SQ_WAVES")):
        v = ratio(a, b)
        if v is not None:
            d[key] = v
    if "TCC_HIT_sum" in c and "TCC_MISS_sum" in c and c["TCC_HIT_sum"] + c["TCC_MISS_sum"] > 0:
        d["l2_hit_rate"] = round(c["TCC_HIT_sum"] / (c["TCC_HIT_sum"] + c["TCC_MISS_sum"]), 4)
    return d


def counters(dirs, kernels=()):
    """{launch shape: {"dispatches": n, "counters": {name: mean per dispatch}, "derived": {...}}}."""
    acc = {}
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                if kernels and not any(k in name for k in kernels):
                    continue
                key = f"{_short(name, 60)} grid {r['Grid_Size']} wg {r['Workgroup_Size']}"
                e = acc.setdefault(key, {})
                e.setdefault(r["Counter_Name"], {})[(d, r["Dispatch_Id"])] = float(r["Counter_Value"])
    out = {}
    for key, e in acc.items():
        means = {c: statistics.mean(v.values()) for c, v in e.items()}
        out[key] = {"dispatches": max(len(v) for v in e.values()),
                    "counters": {c: round(m, 2) for c, m in sorted(means.items())}, "derived": _derive(means)}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--top", type=int, default=20)
    p = sub.add_parser("pmc")
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--kernel", required=True)
    p.add_argument("--bytes", type=int, required=True)
    p.add_argument("--out")
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--kernel", action="append", default=[])
    c.add_argument("--out")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(stats(a.dir, a.top))
        return
    if a.cmd == "counters":
        res = counters(a.dirs, a.kernel)
        print(json.dumps(res, indent=1))
        if a.out:
            json.dump(res, open(a.out, "w"), indent=1)
        return
    res = pmc(a.fetch, a.write, a.kernel, a.bytes)
    res["algorithmic_bytes_per_launch"] = a.bytes
    res["traffic_over_algorithmic"] = round(res["hbm_bytes_per_launch"] / a.bytes, 4)
    print(json.dumps(res, indent=1))
    if a.out:
        json.dump(res, open(a.out, "w"), indent=1)


if __name__ == "__main__":
    sys.exit(main())
