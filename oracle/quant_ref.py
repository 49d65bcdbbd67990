"""numpy restatement of the reference INT4 weight format (test infrastructure, see ``oracle/__init__``).

Follows ``runtime/quant.py`` of the reference:
  * RTN group parameters  ``group_params`` (clip=False branch)      runtime/quant.py:20-39
  * ``quantize`` (RTN, and the clip search of ``group_params``)      runtime/quant.py:17-48
  * ``dequantize``                                                  runtime/quant.py:93-97
  * ``pack`` / ``unpack``                                           runtime/quant.py:100-119
  * ``pack_scale_zero``                                             runtime/quant.py:122-124
  * ``QuantLinear.nbytes``                                          runtime/quant.py:139-140
  * ``dequantize_packed``: unpack + dequantize in torch on any device (the same arithmetic as ``unpack`` and
    ``dequantize``, for weights too large for numpy in a test's time budget)   runtime/quant.py:93-97,114-119

All arithmetic is IEEE float32 with round-half-to-even, exactly the points at which the reference rounds:
``scale = fp16(max((max - min) / 15, 1e-6))`` read back as float32; ``zero = clip(rint(-min / scale), 0, 15)``;
``q = clip(rint(w / scale) + zero, 0, 15)``; dequantized weight ``fp16((q - zero) * scale)`` (one rounding).
Packed word j of a row holds elements 8j..8j+7; element 8j+2i sits at bits [4i, 4i+4) and element 8j+2i+1 at bits
[16+4i, 20+4i); words are stored as signed int32.
"""
import numpy as np

F32 = np.float32
SCALE_FLOOR = F32(1e-6)  # runtime/quant.py:25 clamp(min=1e-6) on a float32 tensor: the float32 nearest 1e-6


def _as_f32(w):
    a = np.asarray(w)
    if a.dtype == np.float16:
        return a.astype(F32)
    if a.dtype != F32:
        raise TypeError(f"expected float16/float32 weights, got {a.dtype}")
    return a


CLIP_GRID = (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7)   # runtime/quant.py:17


def _range_params(lo, hi):
    step = np.maximum((hi - lo) / F32(15), SCALE_FLOOR).astype(F32)
    scale = step.astype(np.float16).astype(F32)
    zero = np.clip(np.rint(-lo / scale), F32(0), F32(15)).astype(F32)
    return scale, zero


def clip_errors(wf, scale, zero):
    """Squared rounding error of each group (float64 sum of the float32 terms (q - zero) * scale - w, squared in
    float32 as runtime/quant.py:33 computes them)."""
    d = ((np.clip(np.rint(wf / scale) + zero, F32(0), F32(15)) - zero) * scale - wf).astype(F32)
    return (d * d).astype(np.float64).sum(axis=-1, keepdims=True)


def group_params(wf, clip=False):
    """wf float32 [..., G] -> (scale, zero) float32 [..., 1] (runtime/quant.py:20-38).

    scale is fp16-representable (rounded to fp16 and read back); zero is an integer in [0, 15]. clip=True shrinks the
    group's [min, max] by the factor of CLIP_GRID (float32, as torch multiplies a float32 tensor by a Python float)
    whose parameters give the smallest squared rounding error, the first factor on ties (the reference's strict
    `err < best`). The errors are summed in float64 here (the reference sums in float32), so this is the exact argmin
    of the reference's float32 terms; the two can differ only where two factors' errors agree within float32
    summation noise."""
    wf = _as_f32(wf)
    lo = wf.min(axis=-1, keepdims=True)
    hi = wf.max(axis=-1, keepdims=True)
    if not clip:
        return _range_params(lo, hi)
    best = None
    for a in CLIP_GRID:
        scale, zero = _range_params((lo * F32(a)).astype(F32), (hi * F32(a)).astype(F32))
        err = clip_errors(wf, scale, zero)
        if best is None:
            best = [err, scale, zero]
        else:
            m = err < best[0]
            best = [np.where(m, err, best[0]), np.where(m, scale, best[1]), np.where(m, zero, best[2])]
    return best[1], best[2]


def quantize(w, group, clip=False):
    """w [N, K] fp16/fp32 -> (q uint8 [N, K], scale fp16 [N, K/G], zero fp16 [N, K/G]) (runtime/quant.py:42-48)."""
    wf = _as_f32(w)
    N, K = wf.shape
    if K % group:
        raise ValueError(f"K={K} is not a multiple of group={group}")
    g = wf.reshape(N, K // group, group)
    scale, zero = group_params(g, clip)
    q = np.clip(np.rint(g / scale) + zero, F32(0), F32(15))
    return (q.reshape(N, K).astype(np.uint8), scale.reshape(N, -1).astype(np.float16),
            zero.reshape(N, -1).astype(np.float16))


def dequantize(q, scale, zero, group):
    """fp16 [N, K] = fp16((q - zero) * scale), one rounding (runtime/quant.py:93-97)."""
    q = np.asarray(q)
    N, K = q.shape
    qf = q.astype(F32).reshape(N, K // group, group)
    z = np.asarray(zero).astype(F32)[..., None]
    s = np.asarray(scale).astype(F32)[..., None]
    return ((qf - z) * s).reshape(N, K).astype(np.float16)


def pack(q):
    """uint8 codes [N, K] (values 0..15) -> int32 words [N, K/8] (runtime/quant.py:100-109)."""
    q = np.asarray(q)
    N, K = q.shape
    if K % 8:
        raise ValueError("K must be a multiple of 8")
    e = q.astype(np.uint32).reshape(N, K // 8, 8)
    word = np.zeros((N, K // 8), dtype=np.uint32)
    for i in range(4):
        word |= e[..., 2 * i] << np.uint32(4 * i)
        word |= e[..., 2 * i + 1] << np.uint32(16 + 4 * i)
    return word.view(np.int32)


def unpack(packed):
    """int32 words [N, W] -> uint8 codes [N, 8W] (runtime/quant.py:112-119)."""
    w = np.ascontiguousarray(packed).view(np.uint32)
    N, W = w.shape
    out = np.empty((N, W, 8), dtype=np.uint8)
    for i in range(4):
        out[..., 2 * i] = (w >> np.uint32(4 * i)) & np.uint32(0xF)
        out[..., 2 * i + 1] = (w >> np.uint32(16 + 4 * i)) & np.uint32(0xF)
    return out.reshape(N, W * 8)


def pack_scale_zero(scale, zero):
    """[N, K/G] scale + zero -> fp16 [N, K/G, 2], (scale, zero) interleaved as a half2 (runtime/quant.py:122-124)."""
    return np.ascontiguousarray(np.stack([np.asarray(scale, np.float16), np.asarray(zero, np.float16)], axis=-1))


def unpack_scale_zero(sz):
    """inverse of ``pack_scale_zero``: fp16 [N, K/G, 2] -> (scale, zero) fp16 [N, K/G]."""
    sz = np.asarray(sz, np.float16)
    return sz[..., 0].copy(), sz[..., 1].copy()


def nbytes(N, K, group):
    """bytes the GEMV reads for one weight: packed int32 + interleaved fp16 scale/zero (runtime/quant.py:139-140)."""
    return (N * K // 8) * 4 + (N * (K // group) * 2) * 2


def gemv_bytes(N, K, group):
    """algorithmic bytes of one W4A16 GEMV: weight + x + y (bench/kernel_bench.py:74)."""
    return nbytes(N, K, group) + 2 * K + 2 * N


# bit offset of element e (0..7) inside its packed word: element 8j+2i at 4i, element 8j+2i+1 at 16+4i
_SHIFTS = tuple(4 * (e // 2) + 16 * (e % 2) for e in range(8))


def dequantize_packed(packed, sz, group):
    """torch int32 packed [N, K/8] + fp16 sz [N, K/G, 2] -> fp16 w_ref [N, K] on packed's device: each nibble is
    extracted at its bit offset (``unpack``), then fp16((q - zero) * scale) with the product in float32 (exact: a
    4-bit integer times an fp16 scale) and one rounding to fp16 (``dequantize``, runtime/quant.py:93-97)."""
    import torch
    N, W = packed.shape
    K = W * 8
    sh = torch.tensor(_SHIFTS, dtype=torch.int32, device=packed.device)
    q = ((packed.unsqueeze(-1) >> sh) & 15).reshape(N, K // group, group).to(torch.float32)
    scale = sz[..., 0].to(torch.float32).unsqueeze(-1)
    zero = sz[..., 1].to(torch.float32).unsqueeze(-1)
    return ((q - zero) * scale).to(torch.float16).reshape(N, K)
