"""INT4 weight format for the W4A16 GEMV, produced on the GPU.

Same format and same numbers as the reference's ``runtime/quant.py`` (RTN ``quantize`` :42-48, ``pack`` :100-109,
``pack_scale_zero`` :122-124): weight W [N, K] -> ``packed`` int32 [N, K/8] (word j holds elements 8j..8j+7; element
8j+2i at bits [4i, 4i+4), element 8j+2i+1 at bits [16+4i, 20+4i)) and ``sz`` fp16 [N, K/G, 2] = (scale, zero) per
(row, group), with scale = fp16((max - min) / 15) (floored at 1e-6), zero = rint(-min / scale) in [0, 15],
q = clamp(rint(w / scale) + zero, 0, 15). The quantize + pack runs as one HIP kernel (dk_quantize_w4), so building
a Llama-3-8B-sized model does not round-trip 16 GB of weights through the host.
"""
import torch

from . import ext


def quantize_pack(w: torch.Tensor, group: int):
    """fp16 CUDA tensor [N, K] -> (packed int32 [N, K/8], sz fp16 [N, K/G, 2]) on the same device."""
    if not w.is_cuda:
        raise RuntimeError("quantize_pack: w must be a CUDA tensor (the format is produced by the HIP kernel)")
    N, K = w.shape
    if K % group:
        raise RuntimeError(f"K={K} is not a multiple of group={group}")
    w16 = w.to(torch.float16).contiguous()
    packed = torch.empty(N, K // 8, dtype=torch.int32, device=w.device)
    sz = torch.empty(N, K // group, 2, dtype=torch.float16, device=w.device)
    ext.load().quantize_w4(w16, packed, sz, group)
    return packed, sz


class QuantLinear:
    """One quantized weight in kernel format (runtime/quant.py:127-140). RTN only: range clipping and GPTQ
    (``clip=True``, ``qsz=``) belong to the calibration producers, which this build does not provide."""

    def __init__(self, w: torch.Tensor, group: int, keep_ref: bool = False, clip: bool = False, qsz=None):
        if clip or qsz is not None:
            raise NotImplementedError("only RTN quantization is produced on the GPU (clip / precomputed codes are not)")
        if keep_ref:
            raise NotImplementedError("the dequantized fp16 reference weight belongs to the CPU oracle, not here")
        self.N, self.K = w.shape
        self.group = group
        self.packed, self.sz = quantize_pack(w, group)
        self.w_ref = None

    def nbytes(self):
        return self.packed.numel() * 4 + self.sz.numel() * 2
