// W4A16 GEMM for prefill on gfx950: Y[M, N] = X[M, K] . dequant(W)[N, K]^T  (fp16 in/out, fp32 accumulation)
//
// The prompt's tokens go through a layer together, so the projections are GEMMs, MFMA-shaped work. The weight format
// is the decode GEMV's (packed int32 [N, K/8], (scale, zero) fp16 [N, K/G, 2]); each weight is dequantized as
// fp16((q - zero) * scale) with one rounding -- the reference's dequantize (runtime/quant.py:93-97) bit for bit:
// (1024 + q) - (1024 + zero), or (64 + q) - (64 + zero) for the nibbles OR-ed in at mantissa bits 4-7, is an exact
// fp16 integer and its fp16 product with the fp16 scale rounds the exact product once -- so every MFMA product is
// exact and the sums are fp32. Epilogue 2 (split-K) writes fp32 partials instead of rows.
//
// Three kernels, chosen by grid size (gemm_w4a16_tile at the end of this file):
//   * register-stationary (K % 128 == 0, G >= 64, a few hundred tiles of 256 weight rows): each wave's 64 weight
//     rows are dequantized in registers straight into the v_mfma_f32_32x32x16_f16 A layout; only the token tile
//     passes through LDS. The fastest form, described at its definition.
//   * wide (K % 64 == 0): weight and token tiles of 64 or 128 both staged in LDS (the weights dequantized on the
//     way), v_mfma_f32_16x16x32_f16, optional K groups inside a workgroup for grids that do not fill the CUs.
//   * the 64 x 64 kernel below (K % 64 == 32): v_mfma_f32_16x16x16_f16 over K chunks of 32.
// Epilogue 0 writes Y [M, N]; epilogue 1 treats the weight rows as interleaved gate / up pairs (row 2i = gate_i, row
// 2i + 1 = up_i, the decode runtime's layout) and writes act[M, N/2] = silu_mul(fp16(gate), fp16(up)), the swiglu
// of the reference's composition with its rounding points.
//
// 64 x 64 kernel: block tile 64 x 64 of Y, four waves of 32 x 32 (2 x 2 MFMA tiles of 16 x 16), K in chunks of 32
// (one 16-byte word group of each weight row; G >= 32 so a chunk never straddles a group). Per chunk the 256 threads
// stage X [64 x 32] (one 16-byte load each) and the dequantized W [64 x 32] (one packed word and its scale/zero each)
// in LDS rows padded to 40 halves (80 B: the 16 rows a wave reads for one operand fall in distinct banks), then each
// wave runs 2 k-steps x 4 MFMAs. The next chunk's global loads are issued before the current chunk's MFMAs (two LDS
// buffers, one barrier per chunk).
//   Operands (lane l = 16 g + c): A = X rows, lane l holds X[row c][k 4g..4g+3]; B = W^T, lane l holds
//   W[col c][k 4g..4g+3]; the accumulator leaves lane l with Y[rows 4g..4g+3][col c].
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

// 8 weights of one packed word -> fp16((q - zero) * scale), in element order, given s2 = (scale, scale), zk = (1024 +
// zero) twice and zs = (64 + zero) twice. Pairs (e0, e1) and (e4, e5) are nibbles 0 and 2 of each 16-bit half: OR-ed
// into the mantissa of fp16 1024 (step 1) they give 1024 + q; pairs (e2, e3) and (e6, e7) are nibbles 1 and 3, and
// OR-ed in place into fp16 64 (step 1/16) they give 64 + q, so one shift (by 8) serves all four pairs. Subtracting
// 1024 + zero or 64 + zero is exact, and the product with the scale rounds the exact (q - zero) * scale once.
// mlo = vgpr_const(0x000F000F), mhi = vgpr_const(0x00F000F0): one v_and_or_b32 per pair.
__device__ __forceinline__ u32x4 dequant8_sz(uint32_t word, f16x2 s2, f16x2 zk, f16x2 zs, uint32_t mlo,
                                             uint32_t mhi) {
  const uint32_t hi = word >> 8;
  const uint32_t p0 = (word & mlo) | 0x64006400u;
  const uint32_t p1 = (word & mhi) | 0x54005400u;
  const uint32_t p2 = (hi & mlo) | 0x64006400u;
  const uint32_t p3 = (hi & mhi) | 0x54005400u;
  u32x4 r;
  r[0] = as_u32((as_f16x2(p0) - zk) * s2);
  r[1] = as_u32((as_f16x2(p1) - zs) * s2);
  r[2] = as_u32((as_f16x2(p2) - zk) * s2);
  r[3] = as_u32((as_f16x2(p3) - zs) * s2);
  return r;
}

// the same from the group's packed (scale, zero) pair (1024 + zero and 64 + zero are exact: zero is an integer in
// [0, 15])
__device__ __forceinline__ u32x4 dequant8(uint32_t word, uint32_t szw, uint32_t mlo, uint32_t mhi) {
  const f16x2 sz = as_f16x2(szw);
  const f16 zk = (f16)1024.0f + sz.y, zs = (f16)64.0f + sz.y;
  return dequant8_sz(word, f16x2{sz.x, sz.x}, f16x2{zk, zk}, f16x2{zs, zs}, mlo, mhi);
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

  const uint32_t mlo = vgpr_const(0x000F000Fu), mhi = vgpr_const(0x00F000F0u);
  auto fetch = [&](int k0, u32x4& xv, uint32_t& wv, uint32_t& sv) {
    xv = *reinterpret_cast<const u32x4*>(xrow + k0);
    wv = __builtin_nontemporal_load(wrow + (k0 >> 3));
    sv = szrow[k0 >> gsh];
  };
  auto stage = [&](int buf, const u32x4& xv, uint32_t wv, uint32_t sv) {
    *reinterpret_cast<u32x4*>(&As[buf][sr][8 * sc]) = xv;
    *reinterpret_cast<u32x4*>(&Bs[buf][sr][8 * sc]) = dequant8(wv, sv, mlo, mhi);
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
// 16 bytes (32 weights), one per thread of the first 2 BN threads, dequantized into LDS. LDS rows are 128 bytes with
// an XOR swizzle of their 16-byte chunks (lds_chunk), which keeps operand reads and both stage patterns free of bank
// conflicts (padded 144-byte rows left the stage writes 2-way conflicted: a third of the LDS cycles). The next chunk's global loads are issued
// before the current chunk's MFMAs (two LDS buffers, one barrier per chunk).
// Workgroup -> tile: workgroups are dealt round-robin to the 8 XCDs, so workgroup b runs on XCD b % 8; the tile
// order is made XCD-major (the b / 8-th tile of XCD b % 8's contiguous range) with the token tiles fastest, so the
// token tiles that share a weight tile run together on one XCD and each weight tile is fetched from HBM once.
constexpr int kWK = 64, kXcds = 8;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// LDS chunk position of 16-byte chunk q (0..7) of row r in the wide kernel's unpadded 128-byte rows. The XOR with
// (r >> 1) & 7 makes every 16-lane group conflict-free on 64 banks: an operand read (16 consecutive rows, one chunk
// each) lands on 2 row parities x 8 distinct positions, the X stage (2 rows x 8 chunks) on both parities, the W stage
// (8 rows x 2 halves, one chunk of each half per store) on 8 distinct positions per parity.
__device__ __forceinline__ int lds_chunk(int r, int q) { return q ^ ((r >> 1) & 7); }

// Phase fence: no memory operation moves across it (the empty asm clobbers memory), so the ring's loads are issued
// where they are written instead of being sunk to their first use, and stay behind the stage's LDS stores. Arithmetic
// may still be scheduled across it, which lets the dequant interleave with the MFMAs.
__device__ __forceinline__ void phase_fence() { asm volatile("" ::: "memory"); }

template <int BN, int BM, int PD, int KG, int EPI>
__global__ void __launch_bounds__(kGemmThreads * KG, KG == 1 ? 2 : 1)
gemm_w4a16_wide(const uint32_t* W, const uint32_t* SZ, const f16* X, f16* Y, int M, int N, int K, int gsh,
                int tiles_m, int tiles) {
  // (no __restrict__: the phase fences below must order these loads, and a fence's memory clobber does not reach
  // memory the compiler knows is only accessed through restrict pointers)
  constexpr int TI = BN / 32, TJ = BM / 32;  // 16 x 16 tiles per wave along n and m
  constexpr int XL = BM * 8 / kGemmThreads;  // 16-byte X loads per thread per chunk
  constexpr int WPT = BN / 32;               // packed W words per thread per chunk (BN x 8 words over 256 threads)
  constexpr int TPR = 8 / WPT;               // threads per W row
  static_assert(XL >= 1 && (WPT == 2 || WPT == 4), "tile shape");
  static_assert(KG == 1 || 2 * BN * kWK * 2 >= TI * TJ * 4 * kGemmThreads * 4, "K-group reduction space");
  // rows of 64 halves = 8 chunks of 16 bytes, chunk q of row r stored at q ^ swz(r) (see lds_chunk)
  __shared__ u32x4 Ws[KG][2][BN][kWK / 8];
  __shared__ u32x4 Xs[KG][2][BM][kWK / 8];
  const int per = gridDim.x / kXcds;
  const int t = (int)(blockIdx.x % kXcds) * per + (int)(blockIdx.x / kXcds);
  if (t >= tiles) return;  // uniform: the grid is rounded up to a multiple of the XCD count
  const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
  // K groups: KG groups of four waves; group kg takes chunks kg, kg + KG, ... with LDS buffers of its own, and the
  // groups' accumulators are summed through LDS at the end (more waves per CU and a KG-times shorter chunk chain
  // for grids that do not fill the CUs)
  const int kg = KG == 1 ? 0 : (int)threadIdx.x / kGemmThreads;
  const int tid = (int)threadIdx.x % kGemmThreads, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int wn = (wave >> 1) * (BN / 2), wm = (wave & 1) * (BM / 2);
  const int KW = K >> 3, NG = K >> gsh;
  // staging roles: X rows tid / 8 + 32 i, 16-byte chunk tid % 8; W row tid / TPR, words WPT (tid % TPR) .. + WPT - 1
  // of the chunk (8 WPT weights, inside one group since G >= 32), every thread loading (no branch in the step)
  const int xr = tid >> 3, xc = tid & 7;
  const f16* xrow[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) xrow[i] = X + (size_t)min(m0 + xr + 32 * i, M - 1) * K + 8 * xc;
  const int wr = tid / TPR, wq = tid % TPR;
  const int wrg = min(n0 + wr, N - 1);
  const uint32_t* wrow = W + (size_t)wrg * KW + WPT * wq;
  const uint32_t* szrow = SZ + (size_t)wrg * NG;

  const int nk = K / kWK;
  u32x4 xv[PD][XL];
  uint32_t wv[PD][WPT], sv[PD];
  // loads are unconditional (threads past 2 BN re-read a valid row, tail fetches re-read the last chunk): loads
  // behind branches make the compiler wait for every outstanding load before a stage, which defeats the ring
  const uint32_t mlo = vgpr_const(0x000F000Fu), mhi = vgpr_const(0x00F000F0u);
  auto fetch = [&](int kc, int slot) {
    const int k0 = min(kc, nk - 1) * kWK;
#pragma unroll
    for (int i = 0; i < XL; ++i) xv[slot][i] = *reinterpret_cast<const u32x4*>(xrow[i] + k0);
    if constexpr (WPT == 4) {
      const u32x4 w4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + (k0 >> 3)));
#pragma unroll
      for (int w = 0; w < 4; ++w) wv[slot][w] = w4[w];
    } else {
      const u32x2 w2 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wrow + (k0 >> 3)));
      wv[slot][0] = w2[0];
      wv[slot][1] = w2[1];
    }
    sv[slot] = szrow[(k0 + 8 * WPT * wq) >> gsh];
  };
  auto stage = [&](int buf, int slot) {
#pragma unroll
    for (int i = 0; i < XL; ++i) Xs[kg][buf][xr + 32 * i][lds_chunk(xr + 32 * i, xc)] = xv[slot][i];
#pragma unroll
    for (int w = 0; w < WPT; ++w)
      Ws[kg][buf][wr][lds_chunk(wr, WPT * wq + w)] = dequant8(wv[slot][w], sv[slot], mlo, mhi);
  };

  f4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // group kg's j-th chunk is kg + KG j (KG divides nk); it lives in register slot j % PD from its fetch until it is staged into the
  // group's LDS buffer j & 1, so its loads are issued PD steps of MFMA work before they are needed
  const int nsteps = nk / KG;
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    fetch(kg + KG * u, u);
    phase_fence();  // slot order = issue order, which the in-order wait counts rely on
  }
  stage(0, 0);
  phase_fence();
  fetch(kg + KG * PD, 0);
  phase_fence();
  __syncthreads();
  // one step: MFMAs of step j from LDS buffer j & 1, stage of step j + 1 from register slot (u + 1) % PD, fetch of
  // step j + 1 + PD into that slot (u = j % PD, a constant wherever this is called)
  auto step = [&](int j, int u) {
    const int buf = j & 1;
    {  // every group has nk / KG steps (the launcher picks KG dividing nk)
#pragma unroll
      for (int ks = 0; ks < kWK / 32; ++ks) {
        h8 a[TI], b[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i)
          a[i] = __builtin_bit_cast(h8, Ws[kg][buf][wn + 16 * i + c][lds_chunk(wn + 16 * i + c, 4 * ks + g)]);
#pragma unroll
        for (int jj = 0; jj < TJ; ++jj)
          b[jj] = __builtin_bit_cast(h8, Xs[kg][buf][wm + 16 * jj + c][lds_chunk(wm + 16 * jj + c, 4 * ks + g)]);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
          for (int jj = 0; jj < TJ; ++jj) acc[i][jj] = mfma32(a[i], b[jj], acc[i][jj]);
        }
      }
    }
    const int nslot = (u + 1) % PD;
    // the stage sits in the MFMAs' basic block, so the scheduler can interleave its dequant and LDS stores with
    // them; the fences keep the fetch after it (the stage then waits only for its own slot's loads, and the other
    // slots' newer loads stay in flight)
    stage(buf ^ 1, nslot);  // step j + 1 (past the end: a copy of the last chunk, never read)
    phase_fence();
    fetch(kg + KG * (j + 1 + PD), nslot);
    phase_fence();
    __syncthreads();
  };
  // whole groups of PD steps in the loop and the remainder after it: a loop body that could exit between its steps
  // and re-enter would leave a path on which the newest loads are a different slot's, and the in-order wait counts
  // would then have to drain everything
  int j0 = 0;
  for (; j0 + PD <= nsteps; j0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) step(j0 + u, u);
  }
#pragma unroll
  for (int u = 0; u + 1 < PD; ++u)
    if (j0 + u < nsteps) step(j0 + u, u);
  if constexpr (KG > 1) {
    // groups 1 .. KG-1 leave their accumulators in their own (now idle) W buffers, lane-major; group 0 adds them
    float* red = reinterpret_cast<float*>(&Ws[kg][0][0][0]);  // 2 BN kWK halves: room for TI TJ 4 floats a lane
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < TI; ++i) {
#pragma unroll
        for (int jj = 0; jj < TJ; ++jj) {
#pragma unroll
          for (int v = 0; v < 4; ++v) red[((i * TJ + jj) * 4 + v) * kGemmThreads + tid] = acc[i][jj][v];
        }
      }
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int q = 1; q < KG; ++q) {
      const float* rq = reinterpret_cast<const float*>(&Ws[q][0][0][0]);
#pragma unroll
      for (int i = 0; i < TI; ++i) {
#pragma unroll
        for (int jj = 0; jj < TJ; ++jj) {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][jj][v] += rq[((i * TJ + jj) * 4 + v) * kGemmThreads + tid];
        }
      }
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

// ---------------------------------------------------------------------------------------------------------------
// Register-stationary weights (K % 128 == 0, G >= 64, grids of a few hundred tiles): every wave owns RW = 64 or 32
// weight rows of the tile (two or one 32-row MFMA tiles) and all of its BM tokens. The weights go from HBM straight into registers --
// lane l = 32 h + r of row tile i loads words 8h .. 8h+7 of row 32 i + r in the 128-wide k chunk (two 16-byte
// loads) -- and are dequantized there, already in the MFMA A layout: no weight passes through LDS and each is
// dequantized once. Only the token tile X [BM x 128] is staged in LDS (rows of 256 bytes, 16-byte chunk q of row t at
// q ^ (t & 15)), written once per chunk and read by all four waves.
//   MFMA: v_mfma_f32_32x32x16_f16. A stream of independent 32x32x16 MFMAs runs at one per 32 clocks per SIMD (the
//   dense fp16 rate), a stream of 16x16x32 ones at about three quarters of that, so the 32 x 32 form carries the
//   kernel; the dequant's vector instructions issue between the MFMAs, one k step ahead of them. k order: in k step s (0..7) of a chunk, lane (h, r) takes word 8h + s of its row
//   (k 64h + 8s .. + 7) and the same eight k of its token row from LDS -- one order for both operands, so the products
//   and their sums are those of the plain order. The accumulator of tile (i, j) leaves lane (h, r) with rows
//   8 q + 4 h + v (q, v = 0..3) of the weight tile for token r: four consecutive outputs of one token per q.
//   LDS traffic: per k step a wave reads BM / 32 token fragments of 1 KB for 2 BM / 32 MFMAs of 32 cycles, 8 bytes
//   per MFMA cycle, 32 per CU cycle with four waves at the full MFMA rate, plus the stage's 16.
// Pipeline per chunk c: compute chunk c (dequant of W(c) in registers, one k step ahead of the MFMAs; X(c) from LDS
// buffer c & 1); halfway through, store the first half of X(c + 1) (loaded a chunk earlier) into the other buffer and
// load its second half; after the MFMAs store that half, issue the loads of X(c + 2)'s first half and W(c + 2), barrier. W, scales and X come in
// through buffer loads (SGPR base and chunk offset, a constant VGPR offset per row), so moving to the next chunk costs
// no vector instruction; the host checks that every offset fits 31 bits. Two workgroups share a CU (accumulators and
// operands in the 256 architectural VGPRs of a wave).
constexpr int kRsK = 128, kRsThreads = 256;
#ifndef RS_AHEAD
#define RS_AHEAD 3
#endif
#ifndef RS_XSPLIT
#define RS_XSPLIT (KS * TJ / 2)
#endif

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, uint32_t bytes) {
  // stride 0 (raw buffer), word 3 = 32-bit data format as the gfx9 family expects for untyped loads
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// EPI 2 (split-K): the grid covers tiles x `splits` work items; item (tile, s) takes the k chunks [s nk / S,
// (s + 1) nk / S) and writes its fp32 partial sums to Y = ws [S][M][N] (float), for gemm_splitk_reduce.
template <int RW, int BM, int EPI>
__global__ void __launch_bounds__(kRsThreads, 2)
gemm_w4a16_rs(const uint32_t* W, const uint32_t* SZ, const f16* X, f16* Y, int M, int N, int K, int gsh,
              int tiles_m, int tiles, int splits) {
  constexpr int TI = RW / 32, TJ = BM / 32, KS = kRsK / 16;
  constexpr int XL = BM * 16 / kRsThreads;  // 16-byte X loads per thread per chunk
  __shared__ u32x4 Xs[2][BM][16];
  const int per = gridDim.x / kXcds;
  const int item = (int)(blockIdx.x % kXcds) * per + (int)(blockIdx.x / kXcds);
  if (item >= tiles * splits) return;  // uniform: the grid is rounded up to a multiple of the XCD count
  // items are split-major with the token tiles fastest, so the tiles that share a weight tile's k range share an XCD
  const int t = item % tiles, split = item / tiles;
  // a ragged last tile is shifted inward (the launcher requires M >= BM and N >= 256), so every row a lane loads is
  // valid; the rows it shares with its neighbour tile are computed by both, bit for bit alike, and stored twice
  const int m0 = min((t % tiles_m) * BM, M - BM), n0 = min((t / tiles_m) * (4 * RW), N - 4 * RW);
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int KW = K >> 3, NG = K >> gsh, nk_all = K / kRsK;
  const int c_lo = split * nk_all / splits, nk = (split + 1) * nk_all / splits - c_lo;  // this item's chunks
  const __amdgpu_buffer_rsrc_t wres = buffer_of(W, (uint32_t)N * (uint32_t)KW * 4u);
  const __amdgpu_buffer_rsrc_t sres = buffer_of(SZ, (uint32_t)N * (uint32_t)NG * 4u);
  const __amdgpu_buffer_rsrc_t xres = buffer_of(X, (uint32_t)M * (uint32_t)K * 2u);
  // one VGPR offset per operand; the row tile (W, scales) and row block (X) go into the SGPR offset. The lane's scale
  // is that of its first k, k0 + 64 h, whose group holds all 64 of its k (G >= 64).
  const uint32_t row = (uint32_t)(n0 + wave * RW + r);
  const uint32_t wo = row * (uint32_t)KW * 4u + 32u * (uint32_t)h;
  const uint32_t so = (row * (uint32_t)NG + (uint32_t)((64 * h) >> gsh)) * 4u;
  // X staging: chunk xq of rows xr + 16 v, stored at chunk xq ^ xr of the row (xr = (xr + 16 v) & 15)
  const int xq = tid & 15, xr = tid >> 4;
  const uint32_t xo = (uint32_t)(m0 + xr) * (uint32_t)K * 2u + 16u * (uint32_t)xq;

  // with 128-token tiles X is staged in two halves of XL / 2 rows per thread, so only half a chunk of it is ever held
  // in registers (the accumulators leave no room for more); W and the scales are held for two chunks, the one
  // computed and the next
  constexpr int NXH = BM >= 128 ? 2 : 1, XH = XL / NXH;
  u32x4 xv[XH], wv[2][TI][2];
  uint32_t sv[2][TI];
  // loads are unconditional (chunks past the end re-read the last one): a load behind a branch would make the
  // compiler drain every outstanding load at the join
  auto fetch_x = [&](int kc, int half) {
    const int k0 = (c_lo + min(kc, nk - 1)) * kRsK;
#pragma unroll
    for (int v = 0; v < XH; ++v)
      xv[v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, xo, 2 * k0 + 32 * K * (v + XH * half), 0));
  };
  auto fetch_w = [&](int kc, int slot) {
    const int k0 = (c_lo + min(kc, nk - 1)) * kRsK;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        wv[slot][i][u] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, wo + 16u * u, (k0 >> 1) + 128 * KW * i, 0));
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
      sv[slot][i] = __builtin_amdgcn_raw_buffer_load_b32(sres, so, ((k0 >> gsh) + 32 * NG * i) * 4, 0);
  };
  auto stage = [&](int buf, int half) {
#pragma unroll
    for (int v = 0; v < XH; ++v) Xs[buf][xr + 16 * (v + XH * half)][xq ^ xr] = xv[v];
  };
  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};
  }
  const uint32_t mlo = vgpr_const(0x000F000Fu), mhi = vgpr_const(0x00F000F0u);
  // MFMAs of one chunk; `mid` (the next chunk's first X half into LDS, its second half's loads) runs after the
  // MFMAs of the first RS_XSPLIT fragments
  auto compute = [&](int buf, int slot, auto&& mid) {
    // the chunk's weight words and scales enter here: without the pin the compiler hoists their first use above the
    // previous chunk's barrier, where waiting for them drains the newer loads as well
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      asm volatile("" : "+v"(wv[slot][i][0]), "+v"(wv[slot][i][1]));
      asm volatile("" : "+v"(sv[slot][i]));
    }
    f16x2 s2[TI], zk[TI], zs[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const f16x2 sz = as_f16x2(sv[slot][i]);
      const f16 a = (f16)1024.0f + sz.y, b = (f16)64.0f + sz.y;  // 1024 + zero and 64 + zero, exact
      s2[i] = f16x2{sz.x, sz.x};
      zk[i] = f16x2{a, a};
      zs[i] = f16x2{b, b};
    }
    // the chunk's KS x TJ token fragments in (k step, token tile) order, each read from LDS RB fragments ahead of
    // its MFMAs so the reads' latency hides behind the MFMAs of the ones before it
    constexpr int NB = KS * TJ, RB = RS_AHEAD;
    h8 b[RB + 1];
    auto read_b = [&](int q) {
      return __builtin_bit_cast(h8, Xs[buf][32 * (q % TJ) + r][(8 * h + q / TJ) ^ (r & 15)]);
    };
    // k step s + 1's weights are dequantized while step s's MFMAs run (two sets of A operands)
    auto dequant = [&](int s, h8 (&a)[TI]) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
        a[i] = __builtin_bit_cast(h8, dequant8_sz(wv[slot][i][s >> 2][s & 3], s2[i], zk[i], zs[i], mlo, mhi));
    };
#pragma unroll
    for (int q = 0; q < RB; ++q) b[q] = read_b(q);
    h8 a[2][TI];
    dequant(0, a[0]);
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int s = q / TJ;
      if (q == RS_XSPLIT) mid();
      if (q + RB < NB) b[(q + RB) % (RB + 1)] = read_b(q + RB);
#pragma unroll
      for (int i = 0; i < TI; ++i) acc[i][q % TJ] = mfma32x32(a[s & 1][i], b[q % (RB + 1)], acc[i][q % TJ]);
      if (q % TJ == 0 && s + 1 < KS) dequant(s + 1, a[(s + 1) & 1]);
    }
  };
  // prologue: X(0) into buffer 0, X(1)'s first half in flight, W(0) and W(1) in flight
  fetch_x(0, 0);
  fetch_w(0, 0);
  phase_fence();
  stage(0, 0);
  phase_fence();
  if constexpr (NXH == 2) {
    fetch_x(0, 1);
    phase_fence();
    stage(0, 1);
    phase_fence();
  }
  fetch_x(1, 0);
  fetch_w(1, 1);
  phase_fence();
  __syncthreads();
  // one chunk c: MFMAs from LDS buffer c & 1 and register slot c & 1; inside them X(c + 1)'s first half goes to the
  // other buffer and its second half is loaded; after them that half is stored, X(c + 2)'s first half and W(c + 2)
  // are loaded (issue order = wait order: each wait leaves the newer loads in flight). With one X part (64-token
  // tiles) all of X(c + 1) is stored after the MFMAs.
  auto step = [&](int kc, int p) {
    compute(p, p, [&] {
      if constexpr (NXH == 2) {
        phase_fence();
        stage(p ^ 1, 0);
        phase_fence();
        fetch_x(kc + 1, 1);
        phase_fence();
      }
    });
    stage(p ^ 1, NXH - 1);
    phase_fence();
    fetch_x(kc + 2, 0);
    fetch_w(kc + 2, p);
    phase_fence();
    __syncthreads();
  };
  // pairs of chunks in the loop, so every chunk's register slot and LDS buffer is a constant
  int kc = 0;
  for (; kc + 2 <= nk; kc += 2) {
    step(kc, 0);
    step(kc + 1, 1);
  }
  if (kc < nk) step(kc, 0);
  // ---- epilogue: lane holds Y[token m0 + 32 j + r][n0 + 64 wave + 32 i + 8 q + 4 h + v] in acc[i][j][4 q + v]
  // Through LDS when the rows allow 16-byte stores (the X buffers are free: the last step ended at a barrier): a
  // direct store of this layout puts each lane on its own token row, 32 rows per store instruction, which kept the
  // memory pipeline busy at the kernel's end; staged, each wave writes its 32-token slices of the tile into its own
  // quarter of the buffers (16-byte chunks XOR-swizzled by token) and stores whole row segments, 16 bytes per lane.
  {
    constexpr int ES = EPI == 2 ? 4 : (EPI == 1 ? 1 : 2);  // output bytes per weight row and token
    constexpr int RB = RW * ES, CPR = RB / 16;              // a token's bytes in the wave's slice, its 16-byte chunks
    static_assert(CPR >= 2 && 32 * CPR % 64 == 0 && 4 * 32 * RB <= (int)sizeof(Xs), "staged epilogue fits");
    const bool co = (reinterpret_cast<uintptr_t>(Y) & 15) == 0 &&  // 16-byte aligned rows (uniform)
                    (EPI == 2 || (EPI == 0 ? (N & 7) == 0 : (N & 15) == 0));
    if (co) {
      uint8_t* reg = reinterpret_cast<uint8_t*>(&Xs[0][0][0]) + wave * 32 * RB;
      const int nw0 = n0 + wave * RW;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int sw = r & (CPR - 1);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x16& a = acc[i][j];
            if constexpr (EPI == 2) {
              const int c = 8 * i + 2 * q + h;
              *reinterpret_cast<float4*>(reg + r * RB + ((c ^ sw) << 4)) =
                  float4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
            } else if constexpr (EPI == 1) {
              // rows (n, n + 1), (n + 2, n + 3) are (gate, up) pairs: act columns (32 i + 8 q + 4 h) / 2 + 0, 1
              const int c = 2 * i + (q >> 1), off = 8 * (q & 1) + 4 * h;
              const f16 a0 = silu_mul((f16)a[4 * q], (f16)a[4 * q + 1]);
              const f16 a1 = silu_mul((f16)a[4 * q + 2], (f16)a[4 * q + 3]);
              *reinterpret_cast<uint32_t*>(reg + r * RB + ((c ^ sw) << 4) + off) = as_u32(f16x2{a0, a1});
            } else {
              const int c = 4 * i + q;
              u32x2 o;
              o[0] = as_u32(f16x2{(f16)a[4 * q], (f16)a[4 * q + 1]});
              o[1] = as_u32(f16x2{(f16)a[4 * q + 2], (f16)a[4 * q + 3]});
              *reinterpret_cast<u32x2*>(reg + r * RB + ((c ^ sw) << 4) + 8 * h) = o;
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the wave's own LDS writes, read by other lanes
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k2 = 0; k2 < 32 * CPR / 64; ++k2) {
          const int idx = lane + 64 * k2, t = idx / CPR, c = idx % CPR;
          const u32x4 v = *reinterpret_cast<const u32x4*>(reg + t * RB + ((c ^ (t & (CPR - 1))) << 4));
          const size_t m = (size_t)(m0 + 32 * j + t);
          if constexpr (EPI == 2)
            *reinterpret_cast<u32x4*>(reinterpret_cast<float*>(Y) + ((size_t)split * M + m) * N + nw0 + 4 * c) = v;
          else if constexpr (EPI == 1)
            *reinterpret_cast<u32x4*>(Y + m * (N >> 1) + (nw0 >> 1) + 8 * c) = v;
          else
            *reinterpret_cast<u32x4*>(Y + m * N + nw0 + 8 * c) = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // reads done before the next slice overwrites
        __builtin_amdgcn_wave_barrier();
      }
      return;
    }
  }
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 7) == 0;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int m = m0 + 32 * j + r;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wave * RW + 32 * i + 8 * q + 4 * h;
        if (n >= N) continue;
        if constexpr (EPI == 2) {  // fp32 partials, N % 4 == 0 (checked by the launcher)
          float* dst = reinterpret_cast<float*>(Y) + ((size_t)split * M + m) * N + n;
          *reinterpret_cast<float4*>(dst) =
              float4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          continue;
        }
        const f16 y0 = (f16)acc[i][j][4 * q], y1 = (f16)acc[i][j][4 * q + 1];
        const f16 y2 = (f16)acc[i][j][4 * q + 2], y3 = (f16)acc[i][j][4 * q + 3];
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
          // rows (n, n + 1) and (n + 2, n + 3) are (gate, up) pairs n / 2 and n / 2 + 1 of act[M, N / 2]
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
}

// Y[m][n] = fp16(sum over s of ws[s][m][n]), s in order (deterministic); four consecutive n per thread (N % 4 == 0).
__global__ void __launch_bounds__(256)
gemm_splitk_reduce(const float* __restrict__ ws, int splits, f16* __restrict__ Y, int MN4) {
  const int i = blockIdx.x * 256 + (int)threadIdx.x;
  if (i >= MN4) return;
  const float4* p = reinterpret_cast<const float4*>(ws) + i;
  float4 a = p[0];
  for (int s = 1; s < splits; ++s) {
    const float4 b = p[(size_t)s * MN4];
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  }
  u32x2 o;
  o[0] = as_u32(f16x2{(f16)a.x, (f16)a.y});
  o[1] = as_u32(f16x2{(f16)a.z, (f16)a.w});
  reinterpret_cast<u32x2*>(Y)[i] = o;
}

// requires M >= BM and N >= 4 RW (the last tile in each direction is shifted inward); splits > 1: epilogue 0, N % 4
// == 0 and a workspace of splits * M * N floats (the partials), reduced by a second launch
template <int RW, int BM>
void launch_rs(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
               int epilogue, int splits, void* ws, hipStream_t st) {
  const int tiles_m = (M + BM - 1) / BM, tiles = tiles_m * ((N + 4 * RW - 1) / (4 * RW));
  const dim3 grid((tiles * splits + kXcds - 1) / kXcds * kXcds);
  const uint32_t* P = (const uint32_t*)packed;
  const uint32_t* S = (const uint32_t*)sz;
  if (splits > 1) {
    hipLaunchKernelGGL((gemm_w4a16_rs<RW, BM, 2>), grid, dim3(kRsThreads), 0, st, P, S, (const f16*)x, (f16*)ws, M, N,
                       K, log2G, tiles_m, tiles, splits);
    if (epilogue == 2) return;  // the partials are the output (their reader sums them)
    const int mn4 = M * (N / 4);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3((mn4 + 255) / 256), dim3(256), 0, st, (const float*)ws, splits,
                       (f16*)y, mn4);
  } else if (epilogue == 1) {
    hipLaunchKernelGGL((gemm_w4a16_rs<RW, BM, 1>), grid, dim3(kRsThreads), 0, st, P, S, (const f16*)x, (f16*)y, M, N, K,
                       log2G, tiles_m, tiles, 1);
  } else {
    hipLaunchKernelGGL((gemm_w4a16_rs<RW, BM, 0>), grid, dim3(kRsThreads), 0, st, P, S, (const f16*)x, (f16*)y, M, N, K,
                       log2G, tiles_m, tiles, 1);
  }
}

#ifndef DK_GEMM_PD
#define DK_GEMM_PD 2
#endif

template <int BN, int BM, int KG, int PD = DK_GEMM_PD>
void launch_wide(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                 int epilogue, hipStream_t st) {
  const int tiles_m = (M + BM - 1) / BM, tiles = tiles_m * ((N + BN - 1) / BN);
  const dim3 grid((tiles + kXcds - 1) / kXcds * kXcds);
  if (epilogue == 1)
    hipLaunchKernelGGL((gemm_w4a16_wide<BN, BM, PD, KG, 1>), grid, dim3(kGemmThreads * KG), 0, st,
                       (const uint32_t*)packed, (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G, tiles_m,
                       tiles);
  else
    hipLaunchKernelGGL((gemm_w4a16_wide<BN, BM, PD, KG, 0>), grid, dim3(kGemmThreads * KG), 0, st,
                       (const uint32_t*)packed, (const uint32_t*)sz, (const f16*)x, (f16*)y, M, N, K, log2G, tiles_m,
                       tiles);
}

}  // namespace

// Tile choice: the register-stationary kernel (K % 128 == 0, G >= 64) in the first of these that gives its number
// of tiles (two workgroups per CU: 512 slots): 256 weight rows x 128 tokens, 320 tiles (returns 42); 128 x 128, 320
// (52); 128 x 64, 160 (51). The 128-row tiles (32 rows per wave) give the narrower shapes their tiles (TinyLlama qkv
// 2560 x 2048 at M 512: 14.0 against 17.3 us on the wide kernel; gate|up 11264 x 2048: 37.1 against 40.3 at 256 x 64;
// Llama-3-8B qkv 6144 x 4096: 40.0 against 41.4 at 256 x 64, 384 tiles against 192, which is why 256 x 64 tiles are
// no longer among the unsplit choices: wherever they reach 160 tiles the 128 x 64 tiling reaches 320); below 160
// they lose to the wide kernel (TinyLlama o and down: 13.8 against 11.4 and 34.2 against 31.3 us at 128 tiles). Otherwise the wide kernel: the largest of 128 x 128, 128 x 64, 64 x 64 whose grid still covers the 256
// CUs, then K groups (KG = 2 or 4 four-wave groups per workgroup; 2 at most for 128 x 64, by LDS) while the grid leaves
// CUs with a single workgroup (returns 10 * tile + KG, tile 3: 128 x 128, 2: 128 x 64, 1: 64 x 64); K % 64 != 0 takes
// the 64 x 64 16x16x16 kernel above (returns 0).
#ifndef DK_GEMM_KG
#define DK_GEMM_KG 0
#endif
#ifndef DK_GEMM_RS
#define DK_GEMM_RS 1
#endif
// Split-K (a workspace given, epilogue 0 or 2 = the partials alone, K % 128 == 0, G >= 64, M >= 64, N >= 256, N % 4 == 0, offsets within 31
// bits): taken when no unsplit register-stationary tiling has its tiles (gemm_w4a16_rs_tile) or K is long (64 chunks
// of 128 or more: Llama-3-8B down 4096 x 14336 at M 512 takes 82 us split 4 ways against 92 unsplit on 128-row
// tiles, while its o 4096 x 4096 takes 28.5 unsplit against 31.6 split). Over 64-token tiles of 256 weight rows, else
// 128: the smallest power-of-two split S in 2..16 whose S x tiles reaches 384 workgroups while every split keeps at
// least 16 of the 128-wide chunks, and only if S x tiles reaches 192. Shorter splits lose: the partials' traffic
// (S x M x N x 4 bytes, written and read back) and the reduce launch outweigh the fuller grid (TinyLlama qkv
// 2560 x 2048 at S 4, 4 chunks per split: 27 against 19 us). Returns S (1: no split) and the rows per wave in *rw.
constexpr int kSplitMinChunks = 16;
int gemm_w4a16_rs_tile(int M, int N, int K, int log2G);

int gemm_w4a16_splits(int M, int N, int K, int log2G, int epilogue, int* rw) {
  *rw = 64;
  if (!DK_GEMM_RS || (epilogue != 0 && epilogue != 2) || K % kRsK != 0 || log2G < 6 || M < 64 || N < 256 || N % 4 != 0 ||
      (long long)N * K > 0x7fffffffLL || (long long)M * K > 0x3fffffffLL)
    return 1;
  const int nk = K / kRsK;
  if (nk < 64 && gemm_w4a16_rs_tile(M, N, K, log2G) != 0) return 1;
  const long long tm = (M + 63) / 64;
  for (int r = 64; r >= 32; r /= 2) {
    const long long tiles = (N + 4 * r - 1) / (4 * r) * tm;
    int s = 2;
    while (s < 16 && tiles * s < 384 && nk / (2 * s) >= kSplitMinChunks) s *= 2;
    if (nk / s >= kSplitMinChunks && tiles * s >= 192) {
      *rw = r;
      return s;
    }
  }
  return 1;
}

size_t gemm_w4a16_workspace_bytes(int M, int N, int K, int log2G, int epilogue) {
  int rw;
  const int s = gemm_w4a16_splits(M, N, K, log2G, epilogue, &rw);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// the unsplit register-stationary tiling (see gemm_w4a16_tile), 0 if none has its tiles
int gemm_w4a16_rs_tile(int M, int N, int K, int log2G) {
  if (!DK_GEMM_RS || K % kRsK != 0 || log2G < 6 || (long long)N * K > 0x7fffffffLL || (long long)M * K > 0x3fffffffLL)
    return 0;
  // weight tiles of 256 (64 rows per wave) and 128 (32 rows per wave), token tiles of 128 and 64
  const long long n_t = (N + 255) / 256, n_t32 = (N + 127) / 128, tm128 = (M + 127) / 128, tm64 = (M + 63) / 64;
  if (M >= 128 && N >= 256 && n_t * tm128 >= 320) return 42;
  if (M >= 128 && N >= 128 && n_t32 * tm128 >= 320) return 52;
  if (M >= 64 && N >= 128 && n_t32 * tm64 >= 160) return 51;
  return 0;
}

int gemm_w4a16_tile(int M, int N, int K, int log2G) {
  if (K % kWK != 0) return 0;
  const int rs = gemm_w4a16_rs_tile(M, N, K, log2G);
  if (rs != 0) return rs;
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  const long long t64m = (long long)((M + 63) / 64) * ((N + 127) / 128);
  const long long t64 = (long long)((M + 63) / 64) * ((N + 63) / 64);
  int tile, kgr;
  if (t128 >= 256) {
    tile = 3;
    kgr = 1;
  } else if (t64m >= 256) {
    tile = 2;
    kgr = t64m > 256 ? 1 : 2;
  } else {
    tile = 1;
    kgr = t64 > 512 ? 1 : (t64 > 256 ? 2 : 4);
  }
  if (DK_GEMM_KG > 0 && tile != 3) kgr = tile == 2 ? (DK_GEMM_KG > 2 ? 2 : DK_GEMM_KG) : DK_GEMM_KG;
  while ((K / kWK) % kgr != 0) kgr >>= 1;  // every K group takes the same number of chunks
  return 10 * tile + kgr;
}

void launch_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                       int epilogue, void* ws, hipStream_t st) {
  if (ws != nullptr) {
    int rw;
    const int splits = gemm_w4a16_splits(M, N, K, log2G, epilogue, &rw);
    if (splits > 1) {
      if (rw == 64) return launch_rs<64, 64>(packed, sz, x, y, M, N, K, log2G, epilogue, splits, ws, st);
      return launch_rs<32, 64>(packed, sz, x, y, M, N, K, log2G, epilogue, splits, ws, st);
    }
  }
  switch (gemm_w4a16_tile(M, N, K, log2G)) {
    case 42: launch_rs<64, 128>(packed, sz, x, y, M, N, K, log2G, epilogue, 1, nullptr, st); return;
    case 52: launch_rs<32, 128>(packed, sz, x, y, M, N, K, log2G, epilogue, 1, nullptr, st); return;
    case 51: launch_rs<32, 64>(packed, sz, x, y, M, N, K, log2G, epilogue, 1, nullptr, st); return;
    case 31: launch_wide<128, 128, 1>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 21: launch_wide<128, 64, 1>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 22: launch_wide<128, 64, 2>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 11: launch_wide<64, 64, 1>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 12: launch_wide<64, 64, 2>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
    case 14: launch_wide<64, 64, 4>(packed, sz, x, y, M, N, K, log2G, epilogue, st); return;
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
