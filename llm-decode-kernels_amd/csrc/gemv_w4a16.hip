// W4A16 GEMV for batch-1 decode on gfx950:  y[N] = dequant(W)[N, K] . x[K]   (fp16 in/out, fp32 accumulation)
//
// Weight format (runtime/quant.py:9-12 of the reference): packed int32 [N, K/8], word j = elements 8j..8j+7 with
// element 8j+2i at bits [4i, 4i+4) and 8j+2i+1 at [16+4i, 20+4i); per (row, group of G) an fp16 (scale, zero) pair.
// Dequantized weight w = (q - zero) * scale.
//
// Streaming kernel. A workgroup owns R consecutive rows; its W waves split the row's K/32 sixteen-byte columns
// (column u = 32 weights), thread t taking columns t, t + 64W, ... For each column a lane loads R x 16 B of nibbles
// (non-temporal), the matching 64 B of x (L2-resident, shared by all rows) and R (scale, zero) words.
//
// Dequant without a per-weight subtract or multiply: OR-ing a nibble into the mantissa of 0x6400 (fp16 1024) gives
// the fp16 value 1024 + q exactly, and masking the nibble one position higher (bits 4..7) gives 1024 + 16 q. One
// v_and_or per pair of weights therefore yields packed fp16 operands for v_dot2_f32_f16 against the fp16 x pairs:
//     dA = sum (1024 + q) x            over the pairs taken from bits 0..3 / 16..19 of w and of w >> 8
//     dB = sum (1024 + 16 q) x         over the pairs taken from bits 4..7 / 20..23 of w and of w >> 8
// With SA, SB the sums of the x values that meet dA resp. dB (computed once per column, shared by the R rows):
//     sum (q - z) x = dA + dB / 16 - (1024 + z) SA - (64 + z) SB
// and the column adds scale * that to the row's fp32 accumulator. All products and the per-column sums are exact or
// fp32-rounded, so the result agrees with the fp32 matvec of the fp16-dequantized weight far inside fp16 output
// precision, and the exact cases (integer x, one-hot x) are reproduced bit for bit.
//
// Per 8 weights: 1 shift + 4 v_and_or + 4 v_dot2 (no dequant multiply), which keeps the ALU well under the HBM time.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)
constexpr uint32_t kLoMask = 0x000F000Fu;
constexpr uint32_t kHiMask = 0x00F000F0u;

// ---------------------------------------------------------------------------------------------------------------
// Stage 0: one wave per row, scalar nibble extraction, per-element dequant rounded to fp16 exactly as
// runtime/quant.py dequantize() does (one rounding of the exact product), fp32 FMA with x.
__global__ void __launch_bounds__(1024)
gemv_w4a16_exact(const uint32_t* __restrict__ W, const uint32_t* __restrict__ SZ, const f16* __restrict__ x,
                 f16* __restrict__ y, int N, int K, int log2G) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= N) return;
  const int words = K >> 3, ng = K >> log2G;
  float acc = 0.f;
  for (int j = lane; j < words; j += kWave) {
    const uint32_t w = W[(size_t)row * words + j];
    const f16x2 sz = as_f16x2(SZ[(size_t)row * ng + ((j << 3) >> log2G)]);
    const float s = (float)sz.x, z = (float)sz.y;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = (float)((w >> (4 * (e >> 1) + 16 * (e & 1))) & 0xFu);
      const float wv = (float)(f16)((q - z) * s);
      acc = fmaf(wv, (float)x[(j << 3) + e], acc);
    }
  }
  acc = group_sum<kWave>(acc);
  if (lane == 0) y[row] = (f16)acc;
}

// ---------------------------------------------------------------------------------------------------------------
// Streaming kernel, R rows per workgroup, blockDim.x = 64 * waves (waves <= 16).
template <int R>
__device__ __forceinline__ void column_fma(const u32x4 (&w)[R], const uint32_t (&szw)[R], const u32x4* __restrict__ xp,
                                           float (&acc)[R]) {
  const u32x4 xc[4] = {xp[0], xp[1], xp[2], xp[3]};
  const f16x2 one = {(f16)1.0f, (f16)1.0f};
  float SA = 0.f, SB = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    SA = dot2(as_f16x2(xc[k].x), one, SA);
    SA = dot2(as_f16x2(xc[k].z), one, SA);
    SB = dot2(as_f16x2(xc[k].y), one, SB);
    SB = dot2(as_f16x2(xc[k].w), one, SB);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float dA = 0.f, dB = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = w[r][k], hi = lo >> 8;
      dA = dot2(as_f16x2((lo & kLoMask) | kMagic), as_f16x2(xc[k].x), dA);
      dB = dot2(as_f16x2((lo & kHiMask) | kMagic), as_f16x2(xc[k].y), dB);
      dA = dot2(as_f16x2((hi & kLoMask) | kMagic), as_f16x2(xc[k].z), dA);
      dB = dot2(as_f16x2((hi & kHiMask) | kMagic), as_f16x2(xc[k].w), dB);
    }
    const f16x2 sz = as_f16x2(szw[r]);
    const float s = (float)sz.x, z = (float)sz.y;
    float c = fmaf(dB, 0.0625f, dA);
    c = fmaf(-(1024.f + z), SA, c);
    c = fmaf(-(64.f + z), SB, c);
    acc[r] = fmaf(s, c, acc[r]);
  }
}

template <int R, bool PF>
__global__ void __launch_bounds__(1024)
gemv_w4a16_stream(const u32x4* __restrict__ W, const uint32_t* __restrict__ SZ, const u32x4* __restrict__ X,
                  f16* __restrict__ y, int N, int U, int gsh) {
  __shared__ float red[16][R];
  const int t = threadIdx.x, nt = blockDim.x;
  const int row0 = blockIdx.x * R;
  const int NG = U >> gsh;
  const u32x4* wrow[R];
  const uint32_t* srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int rr = min(row0 + r, N - 1);  // tail rows: clamp the loads, skip the store
    wrow[r] = W + (size_t)rr * U;
    srow[r] = SZ + (size_t)rr * NG;
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;

  if constexpr (!PF) {
    for (int u = t; u < U; u += nt) {
      u32x4 w[R];
      uint32_t szw[R];
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = load_stream(wrow[r] + u);
#pragma unroll
      for (int r = 0; r < R; ++r) szw[r] = srow[r][u >> gsh];
      column_fma<R>(w, szw, X + 4 * u, acc);
    }
  } else {
    int u = t;
    u32x4 w[R];
    uint32_t szw[R];
    if (u < U) {
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = load_stream(wrow[r] + u);
#pragma unroll
      for (int r = 0; r < R; ++r) szw[r] = srow[r][u >> gsh];
    }
    while (u < U) {
      const int un = u + nt;
      u32x4 wn[R];
      uint32_t szn[R];
      if (un < U) {
#pragma unroll
        for (int r = 0; r < R; ++r) wn[r] = load_stream(wrow[r] + un);
#pragma unroll
        for (int r = 0; r < R; ++r) szn[r] = srow[r][un >> gsh];
      }
      column_fma<R>(w, szw, X + 4 * u, acc);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        w[r] = wn[r];
        szw[r] = szn[r];
      }
      u = un;
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = group_sum<kWave>(acc[r]);
  const int wave = t >> 6, lane = t & 63, nw = nt >> 6;
  if (nw == 1) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane == r && row0 + r < N) y[row0 + r] = (f16)acc[r];
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) red[wave][r] = acc[r];
  }
  __syncthreads();
  if (t < R && row0 + t < N) {
    float v = 0.f;
    for (int i = 0; i < nw; ++i) v += red[i][t];
    y[row0 + t] = (f16)v;
  }
}

template <int R>
void launch_stream(int waves, int pf, const void* packed, const void* sz, const void* x, void* y, int N, int K,
                   int log2G, hipStream_t st) {
  const int U = K >> 5;
  const int blocks = (N + R - 1) / R;
  const int gsh = log2G - 5;
  if (pf)
    hipLaunchKernelGGL((gemv_w4a16_stream<R, true>), dim3(blocks), dim3(64 * waves), 0, st, (const u32x4*)packed,
                       (const uint32_t*)sz, (const u32x4*)x, (f16*)y, N, U, gsh);
  else
    hipLaunchKernelGGL((gemv_w4a16_stream<R, false>), dim3(blocks), dim3(64 * waves), 0, st, (const u32x4*)packed,
                       (const uint32_t*)sz, (const u32x4*)x, (f16*)y, N, U, gsh);
}

}  // namespace

void gemv_default_config(int N, int K, int* R, int* waves, int* pf) {
  const int U = K >> 5;
  int w = (U + 63) / 64;
  if (w > 16) w = 16;
  int r = 4;
  while (r > 1 && (long long)((N + r - 1) / r) * w < 2048) r >>= 1;
  *R = r;
  *waves = w;
  *pf = (U > 64 * w) ? 1 : 0;
}

void launch_gemv_w4a16(int stage, int R, int waves, int pf, const void* packed, const void* sz, const void* x,
                       void* y, int N, int K, int log2G, hipStream_t st) {
  if (stage == 0) {
    const int wpb = waves > 0 ? waves : 4;
    hipLaunchKernelGGL(gemv_w4a16_exact, dim3((N + wpb - 1) / wpb), dim3(64 * wpb), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, N, K, log2G);
    return;
  }
  if (waves <= 0) {
    int r, w, p;
    gemv_default_config(N, K, &r, &w, &p);
    waves = w;
  }
  switch (R) {
    case 1: launch_stream<1>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    case 2: launch_stream<2>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    case 4: launch_stream<4>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    default: launch_stream<8>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
  }
}

}  // namespace dk
