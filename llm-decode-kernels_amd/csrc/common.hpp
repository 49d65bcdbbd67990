// Shared device helpers for the gfx950 (CDNA4, wave64) decode kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dk {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ f16x2 as_f16x2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// 16-byte load that bypasses cache retention: weights and KV rows are read once per token.
__device__ __forceinline__ u32x4 load_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }

// Sum / max over aligned groups of WIDTH consecutive lanes (WIDTH a power of two <= 64); every lane of the group
// ends with the group result.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Reduction over the lanes that share (lane % STRIDE), i.e. xor offsets STRIDE, 2*STRIDE, ..., 32.
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float v) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int STRIDE>
__device__ __forceinline__ float strided_max(float v) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// fp32 dot of two fp16 pairs plus an fp32 accumulator (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// 8 fp16 values of one 16-byte chunk -> fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 h = as_f16x2(v[i]);
    f[2 * i] = (float)h.x;
    f[2 * i + 1] = (float)h.y;
  }
}

}  // namespace dk
