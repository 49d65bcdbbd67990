// INT4 format producer on gfx950: round-to-nearest asymmetric group quantization + nibble packing, bit-identical to
// the reference's runtime/quant.py (group_params RTN branch :20-28, quantize :42-48, pack :100-109,
// pack_scale_zero :122-124):
//     scale = fp16(max((max - min) / 15, 1e-6))        (fp32 arithmetic, read back as fp32)
//     zero  = clamp(rint(-min / scale), 0, 15)
//     q     = clamp(rint(w / scale) + zero, 0, 15)
// rint is round-half-to-even and the divisions are IEEE-correctly rounded, matching torch's fp32 ops.
//
// With clip (group_params clip=True, runtime/quant.py:17-38) the range [min, max] is first shrunk by the factor of
// CLIP_GRID = (1.0, 0.95, ..., 0.7) whose (scale, zero) give the smallest squared rounding error of the group: for each
// factor a (fp32, as torch multiplies an fp32 tensor by a Python float) mn = min * a, mx = max * a, the scale and zero
// above, and err = sum((clamp(rint(w / scale) + zero, 0, 15) - zero) * scale - w)^2 over the group, each term in fp32
// exactly as the reference computes it. The terms are summed in fp64, so the choice (the first factor with the
// smallest error, the reference's strict `err < best`) is the exact argmin of the reference's fp32 terms; the
// reference sums them in fp32, so the two can pick different factors only where two errors agree to fp32 summation
// noise.
//
// One thread per packed word (8 weights, one 16-byte load); the G/8 threads of a group are consecutive lanes of one
// wave (G <= 512) and reduce min / max (and the clip errors) with xor shuffles.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

// torch.clamp semantics: a value equal to a bound (in particular -0.0 against a bound of +0.0) and NaN pass through
// unchanged. fminf / fmaxf would return +0.0 for (-0.0, +0.0) and drop NaN.
__device__ __forceinline__ float clamp_keep_sign(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

constexpr float kClipGrid[7] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f};

// (scale, zero) of a [lo, hi] range: scale = fp16(max((hi - lo) / 15, 1e-6)) read back as fp32, zero =
// clamp(rint(-lo / scale), 0, 15) (a group whose minimum is 0 or a tiny positive value gives -0.0, which the
// reference's clamp keeps).
__device__ __forceinline__ void range_params(float lo, float hi, f16& scale16, float& scale, float& zero) {
  const float step = clamp_keep_sign((hi - lo) / 15.0f, 1e-6f, INFINITY);
  scale16 = (f16)step;
  scale = (float)scale16;
  zero = clamp_keep_sign(rintf(-lo / scale), 0.0f, 15.0f);
}

template <int WPG, bool CLIP>  // words (threads) per group; range clipping
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
  f16 scale16;
  float scale, zero;
  range_params(lo, hi, scale16, scale, zero);
  if constexpr (CLIP) {
    double best = 0.0;
#pragma unroll 1
    for (int i = 0; i < 7; ++i) {
      f16 s16;
      float sc, ze;
      range_params(lo * kClipGrid[i], hi * kClipGrid[i], s16, sc, ze);
      double err = 0.0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (clamp_keep_sign(rintf(v[e] / sc) + ze, 0.0f, 15.0f) - ze) * sc - v[e];
        err += (double)(d * d);
      }
#pragma unroll
      for (int o = WPG / 2; o > 0; o >>= 1) err += __shfl_xor(err, o, kWave);
      if (i == 0 || err < best) {
        best = err;
        scale16 = s16;
        scale = sc;
        zero = ze;
      }
    }
  }
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

template <bool CLIP>
void launch_quantize(const void* w, void* packed, void* sz, int N, int K, int log2G, hipStream_t st) {
  const long long words = (long long)N * (K >> 3);
  const int threads = 256;
  const dim3 grid((unsigned)((words + threads - 1) / threads));
  const f16* wp = (const f16*)w;
  uint32_t* pp = (uint32_t*)packed;
  uint32_t* sp = (uint32_t*)sz;
  switch (log2G) {
    case 5: hipLaunchKernelGGL((quantize_w4_kernel<4, CLIP>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 6: hipLaunchKernelGGL((quantize_w4_kernel<8, CLIP>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 7: hipLaunchKernelGGL((quantize_w4_kernel<16, CLIP>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    case 8: hipLaunchKernelGGL((quantize_w4_kernel<32, CLIP>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
    default: hipLaunchKernelGGL((quantize_w4_kernel<64, CLIP>), grid, dim3(threads), 0, st, wp, pp, sp, N, K); break;
  }
}

}  // namespace

void launch_quantize_w4(const void* w, void* packed, void* sz, int N, int K, int log2G, int clip, hipStream_t st) {
  if (clip)
    launch_quantize<true>(w, packed, sz, N, K, log2G, st);
  else
    launch_quantize<false>(w, packed, sz, N, K, log2G, st);
}

}  // namespace dk
