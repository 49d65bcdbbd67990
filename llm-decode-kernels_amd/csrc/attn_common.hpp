// Decode-attention helpers shared by the split kernels, the prefill kernel and the o projection's combine prologue:
// split count, RoPE of a 16-byte slice, and the 16 x 16 f16 MFMA tile helpers.
#pragma once
#include "common.hpp"

namespace dk {

__device__ __forceinline__ int attn_splits(int ctx, int PS, int max_splits) {
  if (ctx <= 0) return 0;
  const int n = (ctx + PS - 1) / PS;
  return n < max_splits ? n : max_splits;
}

// RoPE of one 8-dim slice c of a head vector x (fp16, D dims): own = x[8c..8c+8), partner = the slice D/2 away.
// out_i = own_i * cos_i + sign * (partner_i * sin_i), sign = -1 in the first half, +1 in the second half; products
// and sums rounded separately (no contraction), result rounded to fp16.
template <int D>
__device__ __forceinline__ u32x4 rope_slice(u32x4 own, u32x4 partner, const float* cs, const float* sn, bool first) {
  // hipcc contracts a*c - b*s into one fma by default (one rounding instead of two), which changes the rotated value
  // in the last bit now and then; the reference rounds both products. The pragma covers the operators written here
  // (not those inside library helpers such as __fmul_rn, whose bodies carry their own contraction flag).
#pragma clang fp contract(off)
  float a[8], b[8];
  unpack8(own, a);
  unpack8(partner, b);
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f16 o2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = 2 * k + e;
      const float p1 = a[i] * cs[i];
      const float p2 = b[i] * sn[i];
      o2[e] = (f16)(first ? p1 - p2 : p1 + p2);
    }
    r[k] = as_u32(f16x2{o2[0], o2[1]});
  }
  return r;
}

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h4 as_h4(uint32_t a, uint32_t b) { return __builtin_bit_cast(h4, u32x2{a, b}); }
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
// over the four 16-lane rows of a wave (lanes c, c + 16, c + 32, c + 48)
__device__ __forceinline__ float rows_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float rows_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

template <int VD>
struct VRow {
  uint32_t w[VD / 2];
};
template <int VD>
__device__ __forceinline__ VRow<VD> load_vrow(const f16* p) {
  VRow<VD> r;
  if constexpr (VD == 4) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else {
    const u32x4 v = load_stream(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = v[i];
  }
  return r;
}

}  // namespace dk
