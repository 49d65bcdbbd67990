"""Kernel timing on one MI355X with cold caches (the role of the reference's bench/timing.py:65-154).

Launches are captured into one hipGraph (``torch.cuda.CUDAGraph``) and replayed, so the measured time is GPU time of
back-to-back kernels, not Python/ctypes launch cost. To keep the weights out of the caches (4 MB L2 per XCD and the
256 MB MALL), each replay walks ``copies`` distinct copies of the operands laid out in one buffer larger than the MALL,
so every launch reads its weights from HBM; the reference flushed L2 with a 16 MB read between iterations instead
(bench/timing.py:28-32), which would not evict a 256 MB MALL.

Per-launch time = time of ``batch`` back-to-back replays (HIP events on the replay stream) / launches in them; the
minimum and median over ``reps`` such samples are reported.
"""
import statistics

import torch

MALL_BYTES = 256 << 20


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
