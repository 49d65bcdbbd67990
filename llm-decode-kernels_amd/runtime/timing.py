"""Kernel timing on one MI355X with cold caches (the role of the reference's bench/timing.py:65-154).

Launches are captured into one hipGraph (``torch.cuda.CUDAGraph``) and replayed, so the measured time is GPU time of
back-to-back kernels, not Python/ctypes launch cost. To keep the weights out of the caches (4 MB L2 per XCD and the
256 MB MALL), each replay walks ``copies`` distinct copies of the operands laid out in one buffer larger than the MALL,
so every launch reads its weights from HBM; the reference flushed L2 with a 16 MB read between iterations instead
(bench/timing.py:28-32), which would not evict a 256 MB MALL.

Per-launch time = time of ``batch`` back-to-back replays (HIP events on the replay stream) / launches in them; the
minimum and median over ``reps`` such samples are reported.

Clock gating (the role of the reference's NVML gating, bench/timing.py:65-80,119-138): the shader clock of an idle
MI355X drops to a few hundred MHz and ramps up only under sustained load, so a window of a few milliseconds that
follows host-side setup can run at a fraction of the full clock. ``windowed_time`` therefore replays the graph back to
back for a warm-up period queued directly ahead of the timed samples (no host synchronisation in between, so the GPU
goes from the warm-up straight into the window), reads the shader clock from sysfs while the timed samples run (between
the first sample's start event and the last sample's end event), and warms again and retries once when the window's
median clock is below ``MIN_SCLK_MHZ``; a window that stays below it is flagged ``throttled``.
"""
import math
import pathlib
import statistics
import time

import torch

MALL_BYTES = 256 << 20
MIN_SCLK_MHZ = 2000          # MI355X's shader clock peaks at 2400 MHz; a window whose median is below this is throttled


def gpu_sysfs_dir(device=0):
    """sysfs directory of the GPU's PCI function (pp_dpm_* clock files, hwmon), or None."""
    try:
        p = torch.cuda.get_device_properties(device)
        d = pathlib.Path(f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0")
        return d if d.exists() else None
    except Exception:                                     # noqa: BLE001 (no device properties: no clock readings)
        return None


def read_clocks(pci):
    """One sample: current shader / memory / fabric clock (the starred line of pp_dpm_*) and edge temperature."""
    out = {}
    if pci is None:
        return out
    for key, f in (("sclk_mhz", "pp_dpm_sclk"), ("mclk_mhz", "pp_dpm_mclk"), ("fclk_mhz", "pp_dpm_fclk")):
        try:
            for line in (pci / f).read_text().splitlines():
                if line.rstrip().endswith("*"):
                    out[key] = int("".join(ch for ch in line.split(":", 1)[1] if ch.isdigit()))
        except (OSError, ValueError, IndexError):
            pass
    for t in sorted(pci.glob("hwmon/hwmon*/temp1_input")):
        try:
            out["temp_c"] = int(t.read_text()) / 1000
        except (OSError, ValueError):
            pass
    return out


def clock_summary(samples):
    """Per-field min / median / max over clock samples, and their count."""
    out = {"samples": len(samples)}
    for k in ("sclk_mhz", "mclk_mhz", "fclk_mhz", "temp_c"):
        v = sorted(s[k] for s in samples if k in s)
        if v:
            out[k] = {"min": v[0], "median": v[len(v) // 2], "max": v[-1]}
    return out


def n_copies(nbytes, min_copies=8, target_bytes=(5 * MALL_BYTES) // 2, max_copies=2048):
    """Copies of an operand set of ``nbytes`` whose total exceeds the MALL 2.5x."""
    return max(min_copies, min(max_copies, -(-target_bytes // max(1, nbytes))))


class ColdCopies:
    """``copies`` 256-byte-aligned copies of a list of tensors, packed into one device buffer."""

    def __init__(self, tensors, copies):
        self.sizes = [t.numel() * t.element_size() for t in tensors]
        self.slot = sum(-(-s // 256) * 256 for s in self.sizes)
        self.copies = copies
        self.buf = torch.empty(self.slot * copies, dtype=torch.uint8, device=tensors[0].device)
        self.views = []
        for c in range(copies):
            off, vs = c * self.slot, []
            for t, s in zip(tensors, self.sizes):
                v = self.buf[off:off + s].view(t.dtype).view(t.shape)
                v.copy_(t)
                vs.append(v)
                off += -(-s // 256) * 256
            self.views.append(vs)

    def __getitem__(self, i):
        return self.views[i % self.copies]


def graph_time(launch, n, reps=5, batch=1):
    """Capture launch(i) for i in range(n) into one graph; returns (min_us, median_us) per launch over reps samples,
    each sample `batch` replays back to back between one pair of events (batch > 1 keeps the GPU busy across replays,
    as in a decode loop: the first launches after the host synchronises with an idle GPU run slower). launch(i) is
    called once eagerly first so that code objects are loaded outside the capture."""
    launch(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(batch):
            g.replay()
        e.record()
        e.synchronize()
        ts.append(s.elapsed_time(e) * 1e3 / (n * batch))
    del g
    return min(ts), statistics.median(ts)


def _capture(launch, n):
    launch(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    return g


def windowed_time(launch, n, reps=7, warm_ms=300.0, window_ms=60.0, pci=None, min_sclk_mhz=MIN_SCLK_MHZ, retries=1):
    """Clock-gated timing of a graph of launch(0) .. launch(n - 1). The graph is replayed back to back for about
    warm_ms of GPU time, then `reps` timed samples of `batch` replays each follow in the same queue (batch sized so the
    samples fill about window_ms); the host reads the clocks from sysfs (`pci`, gpu_sysfs_dir() if None) while the
    samples run. If the window's median shader clock is below min_sclk_mhz the warm-up is doubled and the window
    retaken, up to `retries` times. Returns a dict: min_us / median_us per launch over the samples, samples_us, batch,
    warm_ms, attempts, clocks (clock_summary of the in-window samples) and throttled (median sclk below the bar,
    None when no clock could be read)."""
    pci = gpu_sysfs_dir() if pci is None else pci
    g = _capture(launch, n)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    e.synchronize()
    t_rep = max(s.elapsed_time(e), 1e-3)                 # ms per replay (cold clock: an overestimate)
    batch = max(1, math.ceil(window_ms / reps / t_rep))
    warm = max(1, math.ceil(warm_ms / t_rep))
    res = None
    for attempt in range(1 + retries):
        for _ in range(warm):
            g.replay()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in evs:
            a.record()
            for _ in range(batch):
                g.replay()
            b.record()
        samples = []
        while not evs[-1][1].query():
            if evs[0][0].query():
                c = read_clocks(pci)
                if c:
                    samples.append(c)
            time.sleep(0.0005)
        torch.cuda.synchronize()
        ts = [a.elapsed_time(b) * 1e3 / (n * batch) for a, b in evs]
        clk = clock_summary(samples)
        sclk = clk.get("sclk_mhz", {}).get("median")
        res = {"min_us": min(ts), "median_us": statistics.median(ts), "samples_us": [round(t, 4) for t in ts],
               "batch": batch, "reps": reps, "warm_ms": round(warm * t_rep, 1), "attempts": attempt + 1,
               "clocks": clk, "throttled": None if sclk is None else sclk < min_sclk_mhz}
        if sclk is None or sclk >= min_sclk_mhz:
            break
        warm *= 2
    del g
    return res
