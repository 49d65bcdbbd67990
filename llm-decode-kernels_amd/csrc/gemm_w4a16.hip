// W4A16 GEMM for prefill on gfx950: Y[M, N] = X[M, K] . dequant(W)[N, K]^T  (fp16 in/out, fp32 accumulation)
//
// The prompt's tokens go through a layer together, so the projections are GEMMs, MFMA-shaped work. The weight format
// is the decode GEMV's (packed int32 [N, K/8], (scale, zero) fp16 [N, K/G, 2]); each weight is dequantized on its way
// into LDS as fp16((q - zero) * scale) with one rounding -- the reference's dequantize (runtime/quant.py:93-97) bit
// for bit: (1024 + q) - (1024 + zero) is an exact fp16 integer and its fp16 product with the fp16 scale rounds the
// exact product once -- so every v_mfma_f32_16x16x16_f16 product is exact and the sums are fp32.
//
// Block tile 64 x 64 of Y, four waves of 32 x 32 (2 x 2 MFMA tiles of 16 x 16), K in chunks of 32 (one 16-byte word
// group of each weight row; G >= 32 so a chunk never straddles a group). Per chunk the 256 threads stage X [64 x 32]
// (one 16-byte load each) and the dequantized W [64 x 32] (one packed word and its scale/zero each) in LDS rows padded
// to 40 halves (80 B: the 16 rows a wave reads for one operand fall in distinct banks), then each wave runs 2 k-steps
// x 4 MFMAs. The next chunk's global loads are issued before the current chunk's MFMAs (two LDS buffers, one barrier
// per chunk).
//   Operands (lane l = 16 g + c): A = X rows, lane l holds X[row c][k 4g..4g+3]; B = W^T, lane l holds
//   W[col c][k 4g..4g+3]; the accumulator leaves lane l with Y[rows 4g..4g+3][col c].
// Epilogue 0 writes Y [M, N]; epilogue 1 treats the columns as interleaved gate / up pairs (col 2i = gate_i, col
// 2i + 1 = up_i, the decode runtime's layout) and writes act[M, N/2] = silu_mul(fp16(gate), fp16(up)), the swiglu
// of the reference's composition with its rounding points.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

constexpr int kBM = 64, kBN = 64, kBK = 32, kLdsRow = 40;
constexpr int kGemmThreads = 256;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// 8 weights of one packed word -> fp16((q - zero) * scale), in element order
__device__ __forceinline__ u32x4 dequant8(uint32_t word, uint32_t szw) {
  const f16x2 sz = as_f16x2(szw);
  const f16x2 s2 = {sz.x, sz.x};
  const f16 zb = (f16)1024.0f + sz.y;            // 1024 + zero, exact (zero is an integer in [0, 15])
  const f16x2 z2 = {zb, zb};
  const uint32_t hi = word >> 8;
  // pairs (e0, e1), (e2, e3), (e4, e5), (e6, e7): nibble i of each 16-bit half
  const uint32_t p0 = (word & 0x000F000Fu) | 0x64006400u;
  const uint32_t p1 = ((word >> 4) & 0x000F000Fu) | 0x64006400u;
  const uint32_t p2 = (hi & 0x000F000Fu) | 0x64006400u;
  const uint32_t p3 = ((hi >> 4) & 0x000F000Fu) | 0x64006400u;
  u32x4 r;
  r[0] = as_u32((as_f16x2(p0) - z2) * s2);
  r[1] = as_u32((as_f16x2(p1) - z2) * s2);
  r[2] = as_u32((as_f16x2(p2) - z2) * s2);
  r[3] = as_u32((as_f16x2(p3) - z2) * s2);
  return r;
}

template <int EPI>
__global__ void __launch_bounds__(kGemmThreads)
gemm_w4a16_kernel(const uint32_t* __restrict__ W, const uint32_t* __restrict__ SZ, const f16* __restrict__ X,
                  f16* __restrict__ Y, int M, int N, int K, int gsh) {
  __shared__ __align__(16) f16 As[2][kBM][kLdsRow];
  __shared__ __align__(16) f16 Bs[2][kBN][kLdsRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int KW = K >> 3, NG = K >> gsh;
  // staging roles: X row tid / 4, 16-byte chunk tid % 4; W row tid / 4, packed word tid % 4
  const int sr = tid >> 2, sc = tid & 3;
  const int xm = min(m0 + sr, M - 1), wr = min(n0 + sr, N - 1);
  const f16* xrow = X + (size_t)xm * K + 8 * sc;
  const uint32_t* wrow = W + (size_t)wr * KW + sc;
  const uint32_t* szrow = SZ + (size_t)wr * NG;

  auto fetch = [&](int k0, u32x4& xv, uint32_t& wv, uint32_t& sv) {
    xv = *reinterpret_cast<const u32x4*>(xrow + k0);
    wv = __builtin_nontemporal_load(wrow + (k0 >> 3));
    sv = szrow[k0 >> gsh];
  };
  auto stage = [&](int buf, const u32x4& xv, uint32_t wv, uint32_t sv) {
    *reinterpret_cast<u32x4*>(&As[buf][sr][8 * sc]) = xv;
    *reinterpret_cast<u32x4*>(&Bs[buf][sr][8 * sc]) = dequant8(wv, sv);
  };

  f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 xv;
  uint32_t wv, sv;
  fetch(0, xv, wv, sv);
  stage(0, xv, wv, sv);
  __syncthreads();
  const int nk = K / kBK;
  for (int kc = 0; kc < nk; ++kc) {
    const int buf = kc & 1;
    if (kc + 1 < nk) fetch((kc + 1) * kBK, xv, wv, sv);   // in flight during this chunk's MFMAs
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      h4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const u32x2 av = *reinterpret_cast<const u32x2*>(&As[buf][wm + 16 * i + c][16 * ks + 4 * g]);
        const u32x2 bv = *reinterpret_cast<const u32x2*>(&Bs[buf][wn + 16 * i + c][16 * ks + 4 * g]);
        a[i] = __builtin_bit_cast(h4, av);
        b[i] = __builtin_bit_cast(h4, bv);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
      }
    }
    if (kc + 1 < nk) stage(buf ^ 1, xv, wv, sv);
    __syncthreads();
  }
  // ---- epilogue: lane holds Y[m0 + wm + 16 i + 4 g + v][n0 + wn + 16 j + c]
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 16 * j + c;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm + 16 * i + 4 * g + v;
        const f16 yv = (f16)acc[i][j][v];
        if constexpr (EPI == 0) {
          if (m < M && n < N) Y[(size_t)m * N + n] = yv;
        } else {
          // columns 2i (gate) and 2i + 1 (up) sit in adjacent lanes: the even lane takes its partner's value
          const f16 up = __builtin_bit_cast(f16, (uint16_t)__shfl_down((int)__builtin_bit_cast(uint16_t, yv), 1, kWave));
          if ((c & 1) == 0 && m < M && n + 1 < N) Y[(size_t)m * (N >> 1) + (n >> 1)] = silu_mul(yv, up);
        }
      }
    }
  }
}

}  // namespace

void launch_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                       int epilogue, hipStream_t st) {
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  if (epilogue == 1)
    hipLaunchKernelGGL(gemm_w4a16_kernel<1>, grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G);
  else
    hipLaunchKernelGGL(gemm_w4a16_kernel<0>, grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G);
}

}  // namespace dk
