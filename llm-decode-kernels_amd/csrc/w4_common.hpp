// INT4 column arithmetic shared by the W4A16 GEMV kernels (see the gemv_w4a16.hip header for the derivation of the
// magic-number dequant).
#pragma once
#include "common.hpp"

namespace dk {

constexpr uint32_t kMagic = 0x64006400u;    // fp16 pair (1024, 1024): + q at mantissa bits 0..3
constexpr uint32_t kMagicHi = 0x54005400u;  // fp16 pair (64, 64): + q at mantissa bits 4..7
constexpr uint32_t kLoMask = 0x000F000Fu;
constexpr uint32_t kHiMask = 0x00F000F0u;

// The two nibble masks, held in VGPRs (vgpr_const), so that each pair costs one v_and_or_b32 (mask in the VGPR,
// the magic constant in an SGPR); the kernels build them once, ahead of their loops.
struct NibbleMasks {
  uint32_t lo, hi;
};
__device__ __forceinline__ NibbleMasks nibble_masks() { return {vgpr_const(kLoMask), vgpr_const(kHiMask)}; }
__device__ __forceinline__ f16x2 nibble_pair(uint32_t w, uint32_t mask, uint32_t magic) {
  return as_f16x2((w & mask) | magic);
}

// Sums of the x values that meet the 1024 and the 64 offsets of one column and the constant part of the column's
// result: sum (q - z) x = (d - 1024 SA - 64 SB) - z (SA + SB), so the chain d starts at base = -(1024 SA + 64 SB),
// computed once per column and shared by every row of it, and each row then needs one FMA and the scale multiply.
struct ColumnSums {
  float base, S;
};
__device__ __forceinline__ ColumnSums column_sums(const u32x4 (&xc)[4]) {
  const f16x2 one = {(f16)1.0f, (f16)1.0f};
  float SA = 0.f, SB = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    SA = dot2(as_f16x2(xc[k].x), one, SA);
    SA = dot2(as_f16x2(xc[k].z), one, SA);
    SB = dot2(as_f16x2(xc[k].y), one, SB);
    SB = dot2(as_f16x2(xc[k].w), one, SB);
  }
  return {fmaf(-1024.f, SA, -64.f * SB), SA + SB};
}

// sum (q - z) x of one row over one column, before the scale: the packed word's 32 weights against xc.
__device__ __forceinline__ float column_row(const u32x4& w, float z, const u32x4 (&xc)[4], ColumnSums cs,
                                            NibbleMasks m) {
  float d = cs.base;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = w[k], hi = lo >> 8;
    d = dot2(nibble_pair(lo, m.lo, kMagic), as_f16x2(xc[k].x), d);
    d = dot2(nibble_pair(lo, m.hi, kMagicHi), as_f16x2(xc[k].y), d);
    d = dot2(nibble_pair(hi, m.lo, kMagic), as_f16x2(xc[k].z), d);
    d = dot2(nibble_pair(hi, m.hi, kMagicHi), as_f16x2(xc[k].w), d);
  }
  return fmaf(-z, cs.S, d);
}

}  // namespace dk
