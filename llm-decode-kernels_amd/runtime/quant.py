"""INT4 weight format for the W4A16 GEMV, and its producers.

Same format and same numbers as the reference's ``runtime/quant.py``: weight W [N, K] -> ``packed`` int32 [N, K/8]
(word j holds elements 8j..8j+7; element 8j+2i at bits [4i, 4i+4), element 8j+2i+1 at bits [16+4i, 20+4i)) and
``sz`` fp16 [N, K/G, 2] = (scale, zero) per (row, group), with scale = fp16((max - min) / 15) (floored at 1e-6),
zero = rint(-min / scale) in [0, 15], q = clamp(rint(w / scale) + zero, 0, 15).

Producers:
  * RTN and range-clipped RTN (``quantize_pack(w, group, clip)``): one HIP kernel (dk_quantize_w4) quantizes and
    packs on the GPU, so building a Llama-3-8B-sized model does not round-trip 16 GB of weights through the host.
  * GPTQ (``quantize_gptq``, runtime/quant.py:51-90 of the reference): the column-by-column error feedback through
    the inverse input Hessian, in torch on whatever device the weight lives on (a calibration-time algorithm built
    from Cholesky factorizations and small GEMMs, not a decode kernel), then ``pack_codes`` to the same format.
    ``runtime.gptq.calibrate`` produces the Hessians from calibration tokens.
"""
import torch

from . import ext

# runtime/quant.py:17 of the reference: range factors tried per group by the clipping search
CLIP_GRID = (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7)


def quantize_pack(w: torch.Tensor, group: int, clip: bool = False):
    """fp16 CUDA tensor [N, K] -> (packed int32 [N, K/8], sz fp16 [N, K/G, 2]) on the same device (RTN, or
    range-clipped RTN with clip=True)."""
    if not w.is_cuda:
        raise RuntimeError("quantize_pack: w must be a CUDA tensor (the format is produced by the HIP kernel)")
    N, K = w.shape
    if K % group:
        raise RuntimeError(f"K={K} is not a multiple of group={group}")
    w16 = w.to(torch.float16).contiguous()
    packed = torch.empty(N, K // 8, dtype=torch.int32, device=w.device)
    sz = torch.empty(N, K // group, 2, dtype=torch.float16, device=w.device)
    ext.load().quantize_w4(w16, packed, sz, group, clip)
    return packed, sz


def group_params(wf: torch.Tensor, clip: bool = False):
    """wf fp32 [..., G] -> (scale, zero) fp32 [..., 1] (runtime/quant.py:20-38): the fp16-rounded scale and integer
    zero of the group's [min, max]; with clip, of the range shrunk by the CLIP_GRID factor with the smallest squared
    rounding error (fp32 sums, first factor on ties). Used inside GPTQ, where each group's parameters come from the
    error-updated weights."""
    mn0 = wf.amin(-1, keepdim=True)
    mx0 = wf.amax(-1, keepdim=True)
    best = None
    for a in (CLIP_GRID if clip else (1.0,)):
        mn, mx = mn0 * a, mx0 * a
        scale = ((mx - mn) / 15).clamp(min=1e-6).half().float()
        zero = torch.round(-mn / scale).clamp(0, 15)
        if not clip:
            return scale, zero
        err = ((torch.clamp(torch.round(wf / scale) + zero, 0, 15) - zero) * scale - wf).pow(2).sum(-1, keepdim=True)
        if best is None:
            best = [err, scale, zero]
        else:
            m = err < best[0]
            best = [torch.where(m, err, best[0]), torch.where(m, scale, best[1]), torch.where(m, zero, best[2])]
    return best[1], best[2]


@torch.no_grad()
def quantize_gptq(w: torch.Tensor, H: torch.Tensor, group: int, clip: bool = False, damp: float = 0.01,
                  block: int = 128):
    """GPTQ (Frantar et al. 2022) into the format of ``quantize``: (q uint8 [N, K], scale, zero fp16 [N, K/G]).

    The algorithm of runtime/quant.py:51-90 of the reference: columns are quantized left to right in blocks of
    ``block``; each column's rounding error, divided by the diagonal of the upper Cholesky factor of H^-1, is spread
    over the block's remaining columns, and a block's errors over the later blocks with one GEMM, so the error of the
    layer output X W^T (H = 2 X^T X / n) is minimised rather than the weight error. A group's (scale, zero) are taken
    when the group starts, from the error-updated weights; no activation reordering, so groups stay contiguous and
    the GEMV reads the result unchanged. Dead input channels (H_jj = 0) get zero weights; ``damp`` adds
    damp * mean(diag H) to the diagonal."""
    N, K = w.shape
    if K % group or block % group:
        raise ValueError(f"K={K} and block={block} must be multiples of group={group}")
    W = w.float().clone()
    H = H.float().clone()
    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    W[:, dead] = 0
    H += damp * torch.diag(H).mean() * torch.eye(K, device=H.device)
    Hinv = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(H)), upper=True)
    Q = torch.zeros(N, K, dtype=torch.uint8, device=W.device)
    S = torch.zeros(N, K // group, device=W.device)
    Z = torch.zeros(N, K // group, device=W.device)
    for i1 in range(0, K, block):
        i2 = min(i1 + block, K)
        W1 = W[:, i1:i2].clone()
        Err = torch.zeros_like(W1)
        Hi = Hinv[i1:i2, i1:i2]
        for i in range(i2 - i1):
            c = i1 + i
            if c % group == 0:                # the group lies inside this block (block % group == 0)
                s, z = group_params(W1[:, i:i + group], clip)
                S[:, c // group], Z[:, c // group] = s[:, 0], z[:, 0]
                scale, zero = s[:, 0], z[:, 0]
            col = W1[:, i]
            q = torch.clamp(torch.round(col / scale) + zero, 0, 15)
            Q[:, c] = q.to(torch.uint8)
            e = (col - (q - zero) * scale) / Hi[i, i]
            W1[:, i:] -= e[:, None] * Hi[i, i:][None, :]
            Err[:, i] = e
        W[:, i2:] -= Err @ Hinv[i1:i2, i2:]
    return Q, S.half(), Z.half()


def pack_codes(q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor):
    """Codes uint8 [N, K] and fp16 scale / zero [N, K/G] -> (packed int32 [N, K/8], sz fp16 [N, K/G, 2]) on q's
    device (runtime/quant.py:100-109 pack, :122-124 pack_scale_zero)."""
    N, K = q.shape
    c = q.to(torch.int64).view(N, K // 8, 8)
    word = torch.zeros(N, K // 8, dtype=torch.int64, device=q.device)
    for e in range(8):
        word |= c[..., e] << (4 * (e >> 1) + 16 * (e & 1))
    packed = torch.where(word >= 1 << 31, word - (1 << 32), word).to(torch.int32)
    sz = torch.stack([scale.half(), zero.half()], dim=-1).contiguous()
    return packed, sz


class QuantLinear:
    """One quantized weight in kernel format (runtime/quant.py:127-140): RTN or range-clipped RTN by the HIP producer,
    or precomputed codes ``qsz = (q, scale, zero)`` (e.g. from ``runtime.gptq.calibrate``) packed on the device."""

    def __init__(self, w: torch.Tensor, group: int, keep_ref: bool = False, clip: bool = False, qsz=None):
        if keep_ref:
            raise NotImplementedError("the dequantized fp16 reference weight belongs to the CPU oracle, not here")
        self.N, self.K = w.shape
        self.group = group
        if qsz is not None:
            q, s, z = (t.to(w.device) for t in qsz)
            if q.shape != (self.N, self.K) or s.shape != (self.N, self.K // group) or z.shape != s.shape:
                raise ValueError(f"precomputed codes {tuple(q.shape)} / {tuple(s.shape)} do not fit W {tuple(w.shape)}"
                                 f" at group {group}")
            self.packed, self.sz = pack_codes(q, s, z)
        else:
            self.packed, self.sz = quantize_pack(w, group, clip)
        self.w_ref = None

    def nbytes(self):
        return self.packed.numel() * 4 + self.sz.numel() * 2
