"""The read probe behind the reference's bw_read op (kernels/bindings.cpp:40-43): every 16-byte word of the buffer is
read exactly once, whatever the grid, workgroup size and loads in flight per lane. Checked through the per-wave sums
it stores: with one sink slot per wave they add up (mod 2^32) to the sum of the buffer's 32-bit words, computed here on
the host; a byte past the last whole 16-byte word is not read."""
import numpy as np
import pytest
import torch

from helpers import DEV

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


def word_sum(a):
    return int(a.astype(np.uint64).sum() % (1 << 32))


@pytest.mark.parametrize("nbytes,blocks,threads,unroll", [
    (16, 1, 64, 1),                  # one word
    (16 * 3, 5, 64, 2),              # more workgroups than words: empty slabs
    (16 * 64 * 3 + 16, 5, 64, 2),    # slabs of uneven length, partial last rounds
    (1 << 20, 7, 256, 4),
    (4096 * 16 + 16, 3, 192, 16),    # workgroup size not a power of two
    (31232000, 256, 512, 8),         # the roofline GEMV's byte count
    (31232000, 1024, 1024, 16),
    (31232000, 3812, 512, 1),
])
def test_read_probe_reads_every_word_once(K, nbytes, blocks, threads, unroll):
    g = torch.Generator().manual_seed(nbytes + blocks)
    host = torch.randint(0, 256, (nbytes + 12,), generator=g, dtype=torch.uint8)  # 12 bytes past the read range
    buf = host.to(DEV)
    sink = torch.full((blocks * threads // 64,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
    K.bw_read(buf[:nbytes + 12], sink, blocks, threads, unroll)
    torch.cuda.synchronize()
    words = host[:(nbytes + 12) // 16 * 16].numpy().view(np.uint32)
    assert word_sum(sink.cpu().numpy().view(np.uint32)) == word_sum(words)


def test_read_probe_small_sink_untouched(K):
    """A sink smaller than one slot per wave (the reference callers pass one word) is not written."""
    n = 4 * 64 * 4 * 16
    host = torch.randint(0, 256, (n,), generator=torch.Generator().manual_seed(5), dtype=torch.uint8)
    for words in (1, 3):
        sink = torch.full((words,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
        K.bw_read(host.to(DEV), sink, 4, 64, 4)
        torch.cuda.synchronize()
        assert torch.all(sink.cpu() == 0x5A5A5A5A)
