"""Shared helpers for the parity tests: error metric, seeded inputs built on the CPU (so every box reproduces them),
and oracle-side views of GPU-produced weights."""
import numpy as np
import torch

from oracle import quant_ref as Q

DEV = "cuda"


def err(out, ref):
    """(max_abs, max_rel) with max_rel = max_abs / max|ref| — normwise, as tests/test_kernels.py:30-38."""
    out, ref = out.detach().float().cpu(), ref.detach().float().cpu()
    max_abs = (out - ref).abs().max().item() if out.numel() else 0.0
    return max_abs, max_abs / max(ref.abs().max().item(), 1e-12)


def assert_close(out, ref, tol, what=""):
    max_abs, max_rel = err(out, ref)
    assert np.isfinite(max_abs) and max_rel <= tol, f"{what}: max_abs={max_abs:.3e} max_rel={max_rel:.3e} tol={tol}"
    return max_rel


def gen(seed):
    return torch.Generator().manual_seed(seed)


def make_cache(ctx, n_kv, page, D=64, peaky=1.0, seed=0, extra_pages=3):
    """Paged caches with a random block table over ctx/page + extra pages (tests/test_kernels.py:90-95)."""
    g = gen(seed)
    n_pages = (ctx + page - 1) // page + extra_pages
    kc = (torch.randn(n_pages, n_kv, page, D, generator=g) * peaky).half()
    vc = torch.randn(n_pages, n_kv, page, D, generator=g).half()
    bt = torch.randperm(n_pages, generator=g).int()
    return kc, vc, bt


def dequant_from_gpu(packed, sz, group):
    """fp16 w_ref [N, K] from GPU-produced packed / sz, through the oracle's unpack + dequantize."""
    q = Q.unpack(packed.cpu().numpy())
    s, z = Q.unpack_scale_zero(sz.cpu().numpy())
    return torch.from_numpy(Q.dequantize(q, s, z, group))
