// INT4 format producer on gfx950: round-to-nearest asymmetric group quantization + nibble packing, bit-identical to
// the reference's runtime/quant.py (group_params RTN branch :20-28, quantize :42-48, pack :100-109,
// pack_scale_zero :122-124):
//     scale = fp16(max((max - min) / 15, 1e-6))        (fp32 arithmetic, read back as fp32)
//     zero  = clamp(rint(-min / scale), 0, 15)
//     q     = clamp(rint(w / scale) + zero, 0, 15)
// rint is round-half-to-even and the divisions are IEEE-correctly rounded, matching torch's fp32 ops.
//
// One thread per packed word (8 weights, one 16-byte load); the G/8 threads of a group are consecutive lanes of one
// wave (G <= 512) and reduce min / max with xor shuffles.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

// torch.clamp semantics: a value equal to a bound (in particular -0.0 against a bound of +0.0) and NaN pass through
// unchanged. fminf / fmaxf would return +0.0 for (-0.0, +0.0) and drop NaN.
__device__ __forceinline__ float clamp_keep_sign(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

template <int WPG>  // words (threads) per group
__global__ void __launch_bounds__(256)
quantize_w4_kernel(const f16* __restrict__ w, uint32_t* __restrict__ packed, uint32_t* __restrict__ sz, int N,
                   int K) {
  const int wpr = K >> 3;  // words per row
  const long long words = (long long)N * wpr;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = gid < words;
  const long long wid = live ? gid : words - 1;  // dead tail lanes form whole dead groups (words % WPG == 0)
  const int row = (int)(wid / wpr), j = (int)(wid % wpr);
  const u32x4 raw = *reinterpret_cast<const u32x4*>(w + (size_t)row * K + (size_t)j * 8);
  float v[8];
  unpack8(raw, v);
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    lo = fminf(lo, v[e]);
    hi = fmaxf(hi, v[e]);
  }
#pragma unroll
  for (int o = WPG / 2; o > 0; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o, kWave));
    hi = fmaxf(hi, __shfl_xor(hi, o, kWave));
  }
  const float step = clamp_keep_sign((hi - lo) / 15.0f, 1e-6f, INFINITY);
  const f16 scale16 = (f16)step;
  const float scale = (float)scale16;
  // A group whose minimum is 0 (or a tiny positive value) gives rint(-min / scale) = -0.0, which the reference's
  // clamp keeps: the stored zero point is then fp16 -0.0 (0x8000), reproduced bit for bit here.
  const float zero = clamp_keep_sign(rintf(-lo / scale), 0.0f, 15.0f);
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float qf = clamp_keep_sign(rintf(v[e] / scale) + zero, 0.0f, 15.0f);
    word |= (uint32_t)qf << (4 * (e >> 1) + 16 * (e & 1));
  }
  if (!live) return;
  packed[gid] = word;
  if ((j & (WPG - 1)) == 0) {
    const f16x2 p = {scale16, (f16)zero};
    sz[(size_t)row * (wpr / WPG) + j / WPG] = as_u32(p);
  }
}

}  // namespace

void launch_quantize_w4(const void* w, void* packed, void* sz, int N, int K, int log2G, hipStream_t st) {
  const long long words = (long long)N * (K >> 3);
  const int threads = 256;
  const dim3 grid((unsigned)((words + threads - 1) / threads));
  const f16* wp = (const f16*)w;
  uint32_t* pp = (uint32_t*)packed;
  uint32_t* sp = (uint32_t*)sz;
  switch (log2G) {
    case 5: hipLaunchKernelGGL((quantize_w4_kernel<4>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 6: hipLaunchKernelGGL((quantize_w4_kernel<8>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 7: hipLaunchKernelGGL((quantize_w4_kernel<16>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 8: hipLaunchKernelGGL((quantize_w4_kernel<32>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    default: hipLaunchKernelGGL((quantize_w4_kernel<64>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
  }
}

}  // namespace dk
