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

// ---------------------------------------------------------------------------------------------------------------
// Wide kernel (K % 64 == 0): block tile BN weight rows x BM tokens, K in chunks of 64, four waves as 2 x 2, each
// wave (BN/2) x (BM/2) in 16 x 16 tiles of v_mfma_f32_16x16x32_f16 (gfx950's double-K form: 8 fp16 per lane and
// operand). The weight rows are the A operand, the tokens the B operand, so the accumulator of tile (i, j) leaves
// lane l = 16 g + c with Y^T[rows n 4g..4g+3][token c]: four consecutive outputs of one token row, stored as one
// 8-byte word, and the gate/up pairs of the SwiGLU epilogue ((4g, 4g+1), (4g+2, 4g+3)) inside one lane.
//   Operand k order: lane (g, c) takes halves 8g..8g+7 of its 32-wide k step for both A and B; any k order that is the
//   same for both operands gives the same dot products, so the result does not depend on the instruction's internal
//   assignment of k to lanes.
// Staging per chunk: X [BM x 64] by 16-byte loads (BM / 32 per thread); the W tile [BN x 64] is BN x 2 words of
// 16 bytes (32 weights), one per thread of the first 2 BN threads, dequantized into LDS. Rows are padded to 72 halves
// (144 B) so the 16 rows of one 16-byte operand read fall in distinct banks. The next chunk's global loads are issued
// before the current chunk's MFMAs (two LDS buffers, one barrier per chunk).
// Workgroup -> tile: workgroups are dealt round-robin to the 8 XCDs, so workgroup b runs on XCD b % 8; the tile
// order is made XCD-major (the b / 8-th tile of XCD b % 8's contiguous range) with the token tiles fastest, so the
// token tiles that share a weight tile run together on one XCD and each weight tile is fetched from HBM once.
constexpr int kWK = 64, kWRow = 72, kXcds = 8;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

template <int BN, int BM, int PD, int EPI>
__global__ void __launch_bounds__(kGemmThreads, 2)
gemm_w4a16_wide(const uint32_t* __restrict__ W, const uint32_t* __restrict__ SZ, const f16* __restrict__ X,
                f16* __restrict__ Y, int M, int N, int K, int gsh, int tiles_m, int tiles) {
  constexpr int TI = BN / 32, TJ = BM / 32;  // 16 x 16 tiles per wave along n and m
  constexpr int XL = BM * 8 / kGemmThreads;  // 16-byte X loads per thread per chunk
  static_assert(XL >= 1 && 2 * BN <= kGemmThreads, "tile shape");
  __shared__ __align__(16) f16 Ws[2][BN][kWRow];
  __shared__ __align__(16) f16 Xs[2][BM][kWRow];
  const int per = gridDim.x / kXcds;
  const int t = (int)(blockIdx.x % kXcds) * per + (int)(blockIdx.x / kXcds);
  if (t >= tiles) return;  // uniform: the grid is rounded up to a multiple of the XCD count
  const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int wn = (wave >> 1) * (BN / 2), wm = (wave & 1) * (BM / 2);
  const int KW = K >> 3, NG = K >> gsh;
  // staging roles: X rows tid / 8 + 32 i, 16-byte chunk tid % 8; W row tid / 2, 32-weight half tid % 2
  const int xr = tid >> 3, xc = tid & 7;
  const f16* xrow[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) xrow[i] = X + (size_t)min(m0 + xr + 32 * i, M - 1) * K + 8 * xc;
  const bool wload = tid < 2 * BN;  // uniform per wave
  const int wr = min(tid >> 1, BN - 1), wh = tid & 1;
  const int wrg = min(n0 + wr, N - 1);
  const u32x4* wrow = reinterpret_cast<const u32x4*>(W + (size_t)wrg * KW) + wh;
  const uint32_t* szrow = SZ + (size_t)wrg * NG;

  const int nk = K / kWK;
  u32x4 xv[PD][XL], wv[PD];
  uint32_t sv[PD];
  // loads are unconditional (threads past 2 BN re-read a valid row, tail fetches re-read the last chunk): loads
  // behind branches make the compiler wait for every outstanding load before a stage, which defeats the ring
  auto fetch = [&](int kc, int slot) {
    const int k0 = min(kc, nk - 1) * kWK;
#pragma unroll
    for (int i = 0; i < XL; ++i) xv[slot][i] = *reinterpret_cast<const u32x4*>(xrow[i] + k0);
    wv[slot] = __builtin_nontemporal_load(wrow + (k0 >> 5));
    sv[slot] = szrow[(k0 + 32 * wh) >> gsh];
  };
  auto stage = [&](int buf, int slot) {
#pragma unroll
    for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(&Xs[buf][xr + 32 * i][8 * xc]) = xv[slot][i];
    if (wload) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        *reinterpret_cast<u32x4*>(&Ws[buf][wr][32 * wh + 8 * w]) = dequant8(wv[slot][w], sv[slot]);
    }
  };

  f4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // chunk kc lives in register slot kc % PD from its fetch until it is staged into LDS buffer kc & 1: its loads are
  // issued PD chunks of MFMA work before they are needed
#pragma unroll
  for (int u = 0; u < PD; ++u) fetch(u, u);
  stage(0, 0);
  fetch(PD, 0);
  __syncthreads();
  for (int kc0 = 0; kc0 < nk; kc0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {  // chunk kc = kc0 + u; the slot indices stay compile-time constants
      const int kc = kc0 + u;
      if (kc >= nk) break;
      const int buf = kc & 1;
#pragma unroll
      for (int ks = 0; ks < kWK / 32; ++ks) {
        h8 a[TI], b[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i)
          a[i] = __builtin_bit_cast(h8, *reinterpret_cast<const u32x4*>(&Ws[buf][wn + 16 * i + c][32 * ks + 8 * g]));
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          b[j] = __builtin_bit_cast(h8, *reinterpret_cast<const u32x4*>(&Xs[buf][wm + 16 * j + c][32 * ks + 8 * g]));
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
          for (int j = 0; j < TJ; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
        }
      }
      const int nslot = (u + 1) % PD;  // a constant once the loop is unrolled
      stage(buf ^ 1, nslot);            // chunk kc + 1 (past the end: a copy of the last chunk, never read)
      fetch(kc + 1 + PD, nslot);
      __syncthreads();
    }
  }
  // ---- epilogue: lane holds Y[token m0 + wm + 16 j + c][n0 + wn + 16 i + 4 g + v], v = 0..3
  const bool vec = (N & 3) == 0;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int m = m0 + wm + 16 * j + c;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int n = n0 + wn + 16 * i + 4 * g;
      const f16 y0 = (f16)acc[i][j][0], y1 = (f16)acc[i][j][1], y2 = (f16)acc[i][j][2], y3 = (f16)acc[i][j][3];
      if constexpr (EPI == 0) {
        f16* dst = Y + (size_t)m * N + n;
        if (vec && n + 3 < N) {
          u32x2 o;
          o[0] = as_u32(f16x2{y0, y1});
          o[1] = as_u32(f16x2{y2, y3});
          *reinterpret_cast<u32x2*>(dst) = o;
        } else {
          const f16 yy[4] = {y0, y1, y2, y3};
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < N) dst[v] = yy[v];
        }
      } else {
        // rows (n, n + 1) and (n + 2, n + 3) are (gate, up) pairs i = n / 2 and n / 2 + 1 of act[M, N / 2]
        f16* dst = Y + (size_t)m * (N >> 1) + (n >> 1);
        const f16 a0 = silu_mul(y0, y1), a1 = silu_mul(y2, y3);
        if (vec && n + 3 < N) {
          *reinterpret_cast<uint32_t*>(dst) = as_u32(f16x2{a0, a1});
        } else {
          if (n + 1 < N) dst[0] = a0;
          if (n + 3 < N) dst[1] = a1;
        }
      }
    }
  }
}

#ifndef DK_GEMM_PD
#define DK_GEMM_PD 2
#endif
template <int BN, int BM, int PD = DK_GEMM_PD>
void launch_wide(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                 int epilogue, hipStream_t st) {
  const int tiles_m = (M + BM - 1) / BM, tiles = tiles_m * ((N + BN - 1) / BN);
  const dim3 grid((tiles + kXcds - 1) / kXcds * kXcds);
  if (epilogue == 1)
    hipLaunchKernelGGL((gemm_w4a16_wide<BN, BM, PD, 1>), grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G, tiles_m, tiles);
  else
    hipLaunchKernelGGL((gemm_w4a16_wide<BN, BM, PD, 0>), grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G, tiles_m, tiles);
}

}  // namespace

// Tile choice: the largest of 128 x 128, 128 x 64, 64 x 64 whose grid still fills the 256 CUs (one workgroup of
// 256 threads per CU at least); K % 64 != 0 takes the 64 x 64 16x16x16 kernel above.
int gemm_w4a16_tile(int M, int N, int K) {
  if (K % kWK != 0) return 0;
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  const long long t64m = (long long)((M + 63) / 64) * ((N + 127) / 128);
  if (t128 >= 256) return 3;
  if (t64m >= 256) return 2;
  return 1;
}

void launch_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                       int epilogue, hipStream_t st) {
  switch (gemm_w4a16_tile(M, N, K)) {
    case 3: launch_wide<128, 128>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 2: launch_wide<128, 64>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 1: launch_wide<64, 64>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    default: break;
  }
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  if (epilogue == 1)
    hipLaunchKernelGGL(gemm_w4a16_kernel<1>, grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G);
  else
    hipLaunchKernelGGL(gemm_w4a16_kernel<0>, grid, dim3(kGemmThreads), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G);
}

}  // namespace dk
