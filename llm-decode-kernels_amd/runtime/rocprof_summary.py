"""Summaries of rocprofv3 CSV output (``--output-format csv``) for the measurements reported by bench.py.

    python -m runtime.rocprof_summary stats <rocprof dir> [--top 20]
        per-kernel calls / average / min / max duration and share of GPU time, from *_kernel_stats.csv

    python -m runtime.rocprof_summary pmc --fetch <dir> --write <dir> --kernel <substring> --bytes <B> [--out f.json]
        HBM bytes per dispatch of the kernel whose name contains <substring>, from one FETCH_SIZE pass and one
        WRITE_SIZE pass over ``bench.py --leg gemv``. The counters are scaled by what they read for kernels of known
        size run in the same process (bench.py calibration_leg): bw_read streaming B bytes once (FETCH_SIZE per B read)
        and the last 16 device copies of B bytes (WRITE_SIZE per B written).
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
    rd = kib([r for r in fr if "bw_read_kernel" in r["Kernel_Name"]][-n_cal:])
    cp = kib([r for r in wr if "copyBuffer" in r["Kernel_Name"]][-n_cal:])
    if not (g_f and g_w and rd and cp):
        raise SystemExit("missing dispatches: need the kernel, bw_read and copy dispatches in both passes")
    f_factor = statistics.median(rd) / nbytes
    w_factor = statistics.median(cp) / nbytes
    fetch = statistics.mean(g_f) / f_factor
    write = statistics.mean(g_w) / w_factor
    return {"kernel": kernel, "dispatches": len(g_f), "fetch_size_kib_per_dispatch": round(statistics.mean(g_f) / 1024, 3),
            "write_size_kib_per_dispatch": round(statistics.mean(g_w) / 1024, 3),
            "fetch_factor": round(f_factor, 5), "write_factor": round(w_factor, 5),
            "hbm_read_bytes_per_launch": round(fetch), "hbm_write_bytes_per_launch": round(write),
            "hbm_bytes_per_launch": round(fetch + write)}


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
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(stats(a.dir, a.top))
        return
    res = pmc(a.fetch, a.write, a.kernel, a.bytes)
    res["algorithmic_bytes_per_launch"] = a.bytes
    res["traffic_over_algorithmic"] = round(res["hbm_bytes_per_launch"] / a.bytes, 4)
    print(json.dumps(res, indent=1))
    if a.out:
        json.dump(res, open(a.out, "w"), indent=1)


if __name__ == "__main__":
    sys.exit(main())
