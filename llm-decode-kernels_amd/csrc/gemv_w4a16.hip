// W4A16 GEMV for batch-1 decode on gfx950:  y[N] = dequant(W)[N, K] . x[K]   (fp16 in/out, fp32 accumulation)
//
// Weight format (runtime/quant.py:9-12 of the reference): packed int32 [N, K/8], word j = elements 8j..8j+7 with
// element 8j+2i at bits [4i, 4i+4) and 8j+2i+1 at [16+4i, 20+4i); per (row, group of G) an fp16 (scale, zero) pair.
// Dequantized weight w = (q - zero) * scale. A "column" u of a row is one 16-byte chunk = 32 weights = 8 words; a row
// has U = K / 32 columns.
//
// Dequant without a per-weight subtract or multiply: OR-ing a nibble into the low mantissa bits of 0x6400 (fp16 1024,
// mantissa step 1) gives the fp16 value 1024 + q exactly, and OR-ing the nibble one position higher (bits 4..7) into
// 0x5400 (fp16 64, mantissa step 1/16) gives 64 + q exactly. One v_and_or per pair of weights therefore yields packed
// fp16 operands for v_dot2_f32_f16 against the fp16 x pairs, all accumulated in one fp32 chain:
//     d = sum (1024 + q) x + sum (64 + q) x   (bits 0..3 / 16..19, resp. 4..7 / 20..23, of w and of w >> 8)
// With SA, SB the sums of the x values that meet the 1024 resp. the 64 offsets (computed once per column, shared by
// the R rows):  sum (q - z) x = d - 1024 SA - 64 SB - z (SA + SB),
// and the column adds scale * that to the row's fp32 accumulator. All products and the per-column sums are exact or
// fp32-rounded, so the result agrees with the fp32 matvec of the fp16-dequantized weight far inside fp16 output
// precision, and the exact cases (integer x, one-hot x) are reproduced bit for bit.
// Per 8 weights: 1 shift + 4 v_and_or + 4 v_dot2 (no dequant multiply); per row and column 1 FMA + 1 multiply.
//
// Kernel family (the reference's ladder, kernels/gemv_w4a16.cu:16-130, re-cut for wave64):
//   stage 0  gemv_w4a16_exact   one wave per row, per-element fp16 dequant, fp32 FMA (correctness rung).
//   stage 1  = stage 2 with R = 1.
//   stage 2  gemv_w4a16_rows    each wave owns R consecutive rows and streams all of K: lane l takes columns l,
//                               l + 64, ... (1 KB contiguous per row per wave load), 2^pf column steps of loads in
//                               flight per lane; x is staged once per workgroup in LDS, transposed so that the 64
//                               lanes of a step read consecutive 16-byte words (no bank conflicts). No barrier after
//                               the staging and no LDS reduction: each wave reduces its rows with lane shuffles.
//   stage 3  gemv_w4a16_splitk  the workgroup's waves split K for R rows (x read through the cache), partial sums
//                               reduced through LDS: for narrow N, where whole-row waves would leave CUs idle.
//   stage 4  gemv_w4a16_tile    the workgroup's waves cover K once with a register-resident x slice per lane and
//                               walk 2^pf tiles of R rows, the next tile's loads in flight while the current one is
//                               computed; x is read once per workgroup, row sums by a DPP fold within waves, LDS
//                               across.
// The compiler's scheduler, left alone, issues only two of a tile's weight loads before it starts computing (it keeps
// register pressure low); __builtin_amdgcn_sched_barrier pins every load of a step ahead of its arithmetic.
#include "attn_common.hpp"
#include "common.hpp"
#include "launch.hpp"
#include "w4_common.hpp"

namespace dk {
namespace {

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
// One column (32 weights) of R rows against the column's 32 x values (xc[0..3], 8 fp16 each).
template <int R>
__device__ __forceinline__ void column_fma(const u32x4 (&w)[R], const uint32_t (&szw)[R], const u32x4 (&xc)[4],
                                           NibbleMasks m, float (&acc)[R]) {
  const ColumnSums cs = column_sums(xc);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const f16x2 sz = as_f16x2(szw[r]);
    acc[r] = fmaf((float)sz.x, column_row(w[r], (float)sz.y, xc, cs, m), acc[r]);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Stage 2: wave-owns-rows streaming kernel. blockDim.x = 64 * waves; dynamic LDS = ceil(U / 64) * 4 KB (x,
// transposed: column u's k-th 16-byte word sits at xs[((u >> 6) * 4 + k) * 64 + (u & 63)]).
template <int R, int P>
__global__ void __launch_bounds__(1024)
gemv_w4a16_rows(const u32x4* __restrict__ W, const uint32_t* __restrict__ SZ, const u32x4* __restrict__ X,
                f16* __restrict__ y, int N, int U, int gsh) {
  extern __shared__ u32x4 xs[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int row0 = (blockIdx.x * nw + wave) * R;
  const int NG = U >> gsh;
  const u32x4* wrow[R];
  const uint32_t* srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int rr = min(row0 + r, N - 1);  // tail rows: clamp the loads, skip the store
    wrow[r] = W + (size_t)rr * U;
    srow[r] = SZ + (size_t)rr * NG;
  }

  // Weight loads of the first P steps go out before x is staged: they do not depend on it.
  u32x4 w[P][R];
  uint32_t s[P][R];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = p * kWave + lane;
    if (u < U) {
#pragma unroll
      for (int r = 0; r < R; ++r) w[p][r] = load_stream(wrow[r] + u);
#pragma unroll
      for (int r = 0; r < R; ++r) s[p][r] = srow[r][u >> gsh];
    }
  }
  for (int i = tid; i < 4 * U; i += blockDim.x) {
    const int u = i >> 2, k = i & 3;
    xs[(((u >> 6) << 2) + k) * kWave + (u & 63)] = X[i];
  }
  __syncthreads();

  const NibbleMasks m = nibble_masks();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  const int steps = (U + kWave - 1) / kWave;
  for (int base = 0; base < steps; base += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int st = base + p;
      const int u = st * kWave + lane;
      if (u < U) {
        const u32x4* xp = xs + (st << 2) * kWave + lane;
        const u32x4 xc[4] = {xp[0], xp[kWave], xp[2 * kWave], xp[3 * kWave]};
        column_fma<R>(w[p], s[p], xc, m, acc);
      }
      const int un = u + P * kWave;
      if (un < U) {
#pragma unroll
        for (int r = 0; r < R; ++r) w[p][r] = load_stream(wrow[r] + un);
#pragma unroll
        for (int r = 0; r < R; ++r) s[p][r] = srow[r][un >> gsh];
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum_lane63(acc[r]);
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < N) y[row0 + r] = (f16)acc[r];
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Stage 3: split-K kernel, R rows per workgroup, blockDim.x = 64 * waves (waves <= 16); thread t takes columns
// t, t + 64 * waves, ... Per column the x words, the R weight words and the R (scale, zero) words are all requested
// before any arithmetic (a scheduling barrier keeps the compiler from interleaving them), PF adds one more column of
// loads in flight. Rows are reduced with DPP within each wave, then across waves through LDS.
template <int R, bool PF>
__global__ void __launch_bounds__(1024)
gemv_w4a16_splitk(const u32x4* __restrict__ W, const uint32_t* __restrict__ SZ, const u32x4* __restrict__ X,
                  f16* __restrict__ y, int N, int U, int gsh) {
  __shared__ float red[16][R];
  const int t = threadIdx.x, nt = blockDim.x, lane = t & 63, wave = t >> 6, nw = nt >> 6;
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
  const NibbleMasks m = nibble_masks();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;

  if constexpr (!PF) {
    for (int u = t; u < U; u += nt) {
      u32x4 xc[4], w[R];
      uint32_t szw[R];
#pragma unroll
      for (int k = 0; k < 4; ++k) xc[k] = X[4 * u + k];
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = load_stream(wrow[r] + u);
#pragma unroll
      for (int r = 0; r < R; ++r) szw[r] = srow[r][u >> gsh];
      __builtin_amdgcn_sched_barrier(0);
      column_fma<R>(w, szw, xc, m, acc);
    }
  } else {
    int u = t;
    u32x4 xc[4], w[R];
    uint32_t szw[R];
    if (u < U) {
#pragma unroll
      for (int k = 0; k < 4; ++k) xc[k] = X[4 * u + k];
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = load_stream(wrow[r] + u);
#pragma unroll
      for (int r = 0; r < R; ++r) szw[r] = srow[r][u >> gsh];
    }
    while (u < U) {
      const int un = u + nt;
      u32x4 xn[4], wn[R];
      uint32_t szn[R];
      if (un < U) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xn[k] = X[4 * un + k];
#pragma unroll
        for (int r = 0; r < R; ++r) wn[r] = load_stream(wrow[r] + un);
#pragma unroll
        for (int r = 0; r < R; ++r) szn[r] = srow[r][un >> gsh];
      }
      __builtin_amdgcn_sched_barrier(0);
      column_fma<R>(w, szw, xc, m, acc);
#pragma unroll
      for (int k = 0; k < 4; ++k) xc[k] = xn[k];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        w[r] = wn[r];
        szw[r] = szn[r];
      }
      u = un;
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum_lane63(acc[r]);
  if (nw == 1) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < N) y[row0 + r] = (f16)acc[r];
    }
    return;
  }
  if (lane == 63) {
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

// ---------------------------------------------------------------------------------------------------------------
// Stage 4: row tiles with a stationary x slice. The workgroup's waves cover K once: lane l of wave v owns column
// u = 64 v + l (so U <= 64 * waves) and loads its 32 x values once into registers. The workgroup walks NT tiles of T
// consecutive rows; for each tile every lane requests its column of all T rows at once (T 16-byte loads + T scale /
// zero words), and the loads of later tiles are issued before tile t is computed (2 or 4 tiles in flight, pinned by
// scheduling barriers so the compiler cannot serialise them). The lanes' row partials are folded together over each
// 16-lane DPP row as the tiles finish (fold_rows: T * NT - 1 merging steps for all rows, instead of a wave sum per
// row), the wave quarters and the waves meet in LDS, and T * NT threads finish the rows and store them.
template <int T>
__device__ __forceinline__ void tile_issue(const u32x4* __restrict__ W, const uint32_t* __restrict__ SZ, int row0,
                                           int N, int U, int NG, int uc, int gsh, u32x4 (&w)[T], uint32_t (&s)[T]) {
#pragma unroll
  for (int r = 0; r < T; ++r) w[r] = load_stream(W + (size_t)min(row0 + r, N - 1) * U + uc);
#pragma unroll
  for (int r = 0; r < T; ++r) s[r] = SZ[(size_t)min(row0 + r, N - 1) * NG + (uc >> gsh)];
}

// The lane's partials of one tile's T rows into p[r0 .. r0 + T). Dead lanes (u >= U) hold x = 0, so their partials
// are exactly 0 for finite scales (a non-finite scale of the last column already makes the live lane's row non-finite).
template <int T, int N>
__device__ __forceinline__ void tile_rows(const u32x4 (&w)[T], const uint32_t (&s)[T], const u32x4 (&xc)[4],
                                          ColumnSums cs, NibbleMasks m, int r0, float (&p)[N]) {
#pragma unroll
  for (int r = 0; r < T; ++r) {
    const f16x2 sz = as_f16x2(s[r]);
    // an fma with +0 (v_fma_mix_f32 takes the fp16 scale directly; a multiply would convert it first), equal to the
    // product but for the sign of a zero result
    p[r0 + r] = fmaf((float)sz.x, column_row(w[r], (float)sz.y, xc, cs, m), 0.f);
  }
}

// The x operand of the row-tile kernel, produced per lane for its column u (32 values = 4 x 16 B):
//   kInPlain    x[32u .. 32u+32)
//   kInRmsNorm  the residual + RMSNorm of the reference's add_rmsnorm (kernels/fused_norm.cu:8-54) recomputed by every
//               workgroup: xn = fp16(xi + delta) (xi = x or the row *row of x, the embedding gather), the sum of
//               squares over the workgroup's K values (DPP within waves, LDS across), r = 1 / sqrt(ss / K + eps),
//               value = norm_w * fp16(float(xn) * r). Workgroup 0 writes xn to x_out (a different buffer: every other
//               workgroup still reads xi).
// Split in two: tile_input_load issues the operand loads and tile_input_finish computes the operand. The loads are
// issued before any weight load of the workgroup: a wave's vector loads return in issue order, so operand loads
// issued after the weights would wait behind an HBM round trip and hold back the prologue and the next tile's loads.
enum { kInPlain = 0, kInRmsNorm = 1, kInCombine4 = 2, kInCombine8 = 3, kInCombine16 = 4 };
constexpr bool is_combine(int pro) { return pro >= kInCombine4; }
constexpr int combine_splits(int pro) { return pro == kInCombine4 ? 4 : pro == kInCombine8 ? 8 : 16; }

struct TileRaw {
  u32x4 a[4];  // x / residual
  u32x4 b[4];  // delta
  u32x4 c[4];  // norm weight
};

template <int PRO>
__device__ __forceinline__ void tile_input_load(const GemvInput& in, const void* x, const void* norm_w,
                                                const void* delta, int uc, int K, TileRaw& raw) {
  if constexpr (PRO == kInPlain) {
    const u32x4* X = reinterpret_cast<const u32x4*>(x);
#pragma unroll
    for (int k = 0; k < 4; ++k) raw.a[k] = X[4 * uc + k];
  } else {
    const long long off = in.row != nullptr ? (long long)(*in.row) * (K >> 3) : 0;
    const u32x4* X = reinterpret_cast<const u32x4*>(x) + off;
    const u32x4* Wn = reinterpret_cast<const u32x4*>(norm_w);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      raw.a[k] = X[4 * uc + k];
      raw.c[k] = Wn[4 * uc + k];
    }
    if (delta != nullptr) {
      const u32x4* Dl = reinterpret_cast<const u32x4*>(delta);
#pragma unroll
      for (int k = 0; k < 4; ++k) raw.b[k] = Dl[4 * uc + k];
    }
  }
}

template <int PRO>
__device__ __forceinline__ void tile_input_finish(const GemvInput& in, const void* delta, TileRaw& raw, int uc,
                                                  bool live, int K, float* s_ss, int wave, int gw0, int nw,
                                                  bool writer, u32x4 (&xc)[4]) {
  if constexpr (PRO == kInPlain) {
#pragma unroll
    for (int k = 0; k < 4; ++k) xc[k] = raw.a[k];
  } else {
    u32x4 (&xr)[4] = raw.a;
    if (delta != nullptr) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[k][e] = as_u32(as_f16x2(xr[k][e]) + as_f16x2(raw.b[k][e]));
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(xr[k][e]);
        const float a = (float)h.x, b = (float)h.y;
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
    ss = wave_sum_all(live ? ss : 0.f);
    float tot = ss;
    if (nw > 1) {  // uniform: the row group's waves meet in LDS (a one-wave group has its total already)
      if ((threadIdx.x & 63) == 0) s_ss[wave] = ss;
      __syncthreads();
      tot = 0.f;
      for (int i = 0; i < nw; ++i) tot += s_ss[gw0 + i];
    }
    const float r = 1.0f / sqrtf(tot / (float)K + in.eps);
    if (writer && in.x_out != nullptr && live) {
#pragma unroll
      for (int k = 0; k < 4; ++k) store_through16(in.x_out, (4 * uc + k) * 16, xr[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(xr[k][e]);
        const f16x2 hn = {(f16)((float)h.x * r), (f16)((float)h.y * r)};
        xc[k][e] = as_u32(as_f16x2(raw.c[k][e]) * hn);
      }
    }
  }
  if (!live) {
#pragma unroll
    for (int k = 0; k < 4; ++k) xc[k] = u32x4{0u, 0u, 0u, 0u};
  }
}

// The attention-combine operand (prologues kInCombine4/8/16, MS = 4, 8 or 16 >= max_splits): the o projection
// merges the split kernel's partials itself instead of a separate combine launch (the log-sum-exp merge of
// kernels/paged_attention.cu:368-427). Thread t of the workgroup takes the 8 values 8t .. 8t + 8 of x (head h, dims
// d0 .. d0 + 8): x = sum_s w_s o_s / sum_s w_s l_s with w_s = e^(m_s - M), M the largest live m_s; with at most one
// live split (or none, when the RoPE split kernel skipped an out-of-range position) x is the attention output the
// split kernel wrote itself. The loads of all max_splits splits (<= MS) go out before the position is known, then
// splits past the live count are dropped by select. The workgroup leaves x in LDS; each lane then
// reads its 32-value column from there.
template <int MS>
struct CombineRaw {
  float4 o[MS][2];
  float m[MS], l[MS];
  u32x4 a;
};

template <int MS>
__device__ __forceinline__ void combine_load(const GemvCombine& c, const float* o_part, const float* m_part,
                                             const float* l_part, int K, CombineRaw<MS>& raw) {
  const int chunk = min((int)threadIdx.x, (K >> 3) - 1);
  const int D = 1 << c.log2D;
  const int h = (chunk << 3) >> c.log2D, d0 = (chunk << 3) & (D - 1);
  const size_t hb = (size_t)h * c.max_splits;
#pragma unroll
  for (int s = 0; s < MS; ++s) {
    raw.o[s][0] = raw.o[s][1] = float4{0.f, 0.f, 0.f, 0.f};
    raw.m[s] = -INFINITY;
    raw.l[s] = 0.f;
    if (s < c.max_splits) {  // uniform: no load for the batch's slots past the buffer's splits
      const size_t hs = hb + s;
      const float4* op = reinterpret_cast<const float4*>(o_part + hs * D + d0);
      raw.o[s][0] = op[0];
      raw.o[s][1] = op[1];
      raw.m[s] = m_part[hs];
      raw.l[s] = l_part[hs];
    }
  }
  raw.a = reinterpret_cast<const u32x4*>(c.attn)[chunk];
}

template <int MS>
__device__ __forceinline__ void combine_finish(const GemvCombine& c, const CombineRaw<MS>& raw, int pos, int K,
                                               u32x4* xs) {
  const bool skip = c.max_pos > 0 && (pos < 0 || pos >= c.max_pos);
  const int ctx = (int)min((long long)pos + 1, (long long)c.cap);
  const int nsplit = skip ? 0 : attn_splits(ctx, c.part_size, c.max_splits);
  u32x4 xv = raw.a;
  if (nsplit > 1) {
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < MS; ++s) M = s < nsplit ? fmaxf(M, raw.m[s]) : M;
    float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MS; ++s) {
      // splits past the live count are replaced, not weighted by 0: their partials are stale or were never written
      // (0 * NaN would poison the sums)
      const bool on = s < nsplit;
      const float ms = on ? raw.m[s] : -INFINITY;
      const float w = ms == -INFINITY ? 0.f : __expf(ms - M);
      L = fmaf(w, on ? raw.l[s] : 0.f, L);
      const float v[8] = {raw.o[s][0].x, raw.o[s][0].y, raw.o[s][0].z, raw.o[s][0].w,
                          raw.o[s][1].x, raw.o[s][1].y, raw.o[s][1].z, raw.o[s][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(w, on ? v[e] : 0.f, acc[e]);
    }
    // o / L, divided as the reference's combine divides (kernels/paged_attention.cu:381); no live weight: 0
#pragma unroll
    for (int k = 0; k < 4; ++k)
      xv[k] = as_u32(L > 0.f ? f16x2{(f16)(acc[2 * k] / L), (f16)(acc[2 * k + 1] / L)} : f16x2{(f16)0.f, (f16)0.f});
  }
  if ((int)threadIdx.x < (K >> 3)) xs[threadIdx.x] = xv;
}

// The output of the row-tile kernel:
//   kOutRows    y[n] = fp16(row sum n)                                      (y has N entries)
//   kOutSwiglu  the rows are interleaved gate / up pairs (row 2i = gate_i, row 2i + 1 = up_i) and
//               y[i] = silu_mul(fp16(row 2i), fp16(row 2i + 1))              (y has N / 2 entries)
//               = swiglu (kernels/fused_swiglu.cu:7-21) of the gate|up GEMV's output, rounded exactly as the two
//               separate ops round it. Needs an even tile (T * NT) so that a pair never straddles two workgroups.
//   kOutRope    the qkv projection with its rows stored per head as rotation pairs (row 2j of head h = row h*D + j,
//               row 2j + 1 = row h*D + j + D/2 of the reference's layout) followed by the reference's rope_append
//               (kernels/rope.cu, as restated by rope_append_kernel): y receives the qkv vector in the reference's
//               order with q rotated and k, v as projected; rotated k and v go to the cache slot of *pos. Nothing
//               is rotated or appended when *pos is outside [0, max_pos); no append when its page is unmapped.
enum { kOutRows = 0, kOutSwiglu = 1, kOutRope = 2 };

// (lo, hi) = (a c - b s, b c + a s) with both products rounded, as the reference's RoPE rounds them.
__device__ __forceinline__ void rope_rotate(f16 a16, f16 b16, float c, float s, f16& lo, f16& hi) {
#pragma clang fp contract(off)
  const float a = (float)a16, b = (float)b16;
  const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
  lo = (f16)(ac - bs);
  hi = (f16)(bc + as);
}

// Total of row `row` of a row group: its partials from the four quarters of each of the group's nw waves.
template <int NR>
__device__ __forceinline__ float row_total(const float* red, int gw0, int nw, int row) {
  float acc = 0.f;
  for (int i = 0; i < nw; ++i) {
    const float* q = red + (gw0 + i) * 4 * NR + row;
    acc += (q[0] + q[NR]) + (q[2 * NR] + q[3 * NR]);
  }
  return acc;
}

// Weight tiles in flight per wave (the buffers of the pipeline): 2, or 4 for walks of 8 tiles of at most 2 rows
// (4096 x 14336 at 2-row tiles: 7.02 against 7.13 us; 3-4 tiles measured no better at shorter walks, all 8 at once
// 7.36, and 4 tiles of 4 or 8 rows spill registers).
constexpr int tile_depth(int t, int nt) { return nt >= 8 && t <= 2 ? 4 : nt < 2 ? nt : 2; }

// Pipeline: operand loads, then the weight loads of tiles 0 .. DP - 1 (DP = tile_depth), then the operand (waits for
// the operand loads only), then for each tile t: compute it from its buffer, refill that buffer with tile t + DP and
// fold the tile's rows. DP tiles are in flight from the first instruction on.
// A workgroup holds blockDim / (64 nw) independent row groups of nw = ceil(U / 64) waves each (group g takes the
// workgroup's g-th run of T * NT rows): at small K a group is one wave, and several groups per workgroup cost fewer
// workgroup dispatches than one single-wave workgroup per row tile.
// `groups` (row groups per workgroup, blockDim / (64 nw)) comes from the host: the kernel's address arithmetic ahead
// of its first load holds no integer division (two of them, at 20-30 dependent instructions each, cost 0.2 us per
// launch at 4096 x 14336). The arguments that the first loads need (weights, scales, the prologue's operands, the
// sizes) come first, so that they are preloaded into scalar registers at launch (-amdgpu-kernarg-preload-count):
// reading them from the kernel-argument segment was one more dependent round trip ahead of the first load (0.2 us
// per launch). The prologue's operands: op0 = x (the residual or embedding table for the norm), op1 = the norm
// weight, op2 = delta (may be null); for the combine prologue o_part, m_part and l_part.
template <int T, int NT, int PRO, int EPI>
__global__ void __launch_bounds__(is_combine(PRO) ? 64 * kGemvCombineMaxWarps : 1024)
gemv_w4a16_tile(const u32x4* __restrict__ W, const uint32_t* __restrict__ SZ, const void* op0, int N, int U, int gsh,
                int groups, const void* op1, const void* op2, f16* __restrict__ y, const GemvInput in) {
  static_assert(EPI == kOutRows || (T * NT) % 2 == 0, "gate/up and rotation pairs need an even row tile");
  static_assert(!is_combine(PRO) || EPI == kOutRows, "the combine prologue feeds the plain epilogue");
  // row partials: [wave][quarter of the wave][row] (the quarters of a row fold, summed when the rows are finished)
  __shared__ float red[16 * 4 * T * NT];
  __shared__ float s_ss[16];
  __shared__ u32x4 xs[is_combine(PRO) ? kGemvCombineMaxWarps * 64 : 1];   // combine: x, 8 values per thread
  const int nw = (U + kWave - 1) / kWave;  // waves of one row group
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int grp = 0;                                  // row group: wave / nw, by comparisons (groups <= 16)
  for (int g = 1; g < groups; ++g) grp += wave >= g * nw ? 1 : 0;
  const int gw0 = grp * nw;                     // its first wave
  const int tid = threadIdx.x - gw0 * kWave;    // thread within the row group
  const int u = (wave - gw0) * kWave + lane;
  const bool live = u < U;
  const int uc = live ? u : U - 1;  // dead lanes load a valid column and contribute 0
  const int base = (blockIdx.x * groups + grp) * T * NT;
  const int NG = U >> gsh;
  int rpos = -1;
  if constexpr (EPI == kOutRope) rpos = *in.rope.pos;
  int cpos = 0;
  if constexpr (is_combine(PRO)) cpos = *in.comb.pos;

  TileRaw raw;
  CombineRaw<is_combine(PRO) ? combine_splits(PRO) : 1> craw;
  if constexpr (is_combine(PRO))
    combine_load(in.comb, static_cast<const float*>(op0), static_cast<const float*>(op1),
                 static_cast<const float*>(op2), U << 5, craw);
  else
    tile_input_load<PRO>(in, op0, op1, op2, uc, U << 5, raw);
  constexpr int DP = tile_depth(T, NT);
  u32x4 w[DP][T];
  uint32_t sz[DP][T];
#pragma unroll
  for (int d = 0; d < DP; ++d) tile_issue<T>(W, SZ, base + d * T, N, U, NG, uc, gsh, w[d], sz[d]);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 xc[4];
  if constexpr (is_combine(PRO)) {
    combine_finish(in.comb, craw, cpos, U << 5, xs);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) xc[k] = live ? xs[4 * uc + k] : u32x4{0u, 0u, 0u, 0u};
  } else {
    tile_input_finish<PRO>(in, op2, raw, uc, live, U << 5, s_ss, wave, gw0, nw, blockIdx.x == 0 && grp == 0, xc);
  }
  const ColumnSums cs = column_sums(xc);
  const NibbleMasks m = nibble_masks();
  // rotation-pair operands of the RoPE epilogue, requested before the tiles are computed
  const int hb = EPI == kOutRope ? in.rope.log2D - 1 : 0;
  const int rp = (base >> 1) + tid, rhead = rp >> hb, ri = rp & ((1 << hb) - 1);
  const bool rvalid = rpos >= 0 && rpos < in.rope.max_pos;
  float rc = 1.f, rs = 0.f;
  int rpage = -1;
  if constexpr (EPI == kOutRope) {
    if (tid < T * NT / 2 && 2 * rp + 1 < N && rvalid) {
      if (rhead < in.rope.n_q + in.rope.n_kv) {
        rc = in.rope.cos_t[((size_t)rpos << hb) + ri];
        rs = in.rope.sin_t[((size_t)rpos << hb) + ri];
      }
      const int lp = rpos >> in.rope.log2P;
      if (lp < in.rope.n_bt) {
        rpage = in.rope.bt[lp];
        if (rpage < 0 || rpage >= in.rope.n_pages) rpage = -1;
      }
    }
  }
  constexpr int NR = T * NT;  // rows of the row group, folded over each 16-lane row as the tiles finish
  const FoldLane fl = fold_lane(lane, NR);
  float p[NR];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tile_rows<T, NR>(w[t % DP], sz[t % DP], xc, cs, m, t * T, p);
    if (t + DP < NT) tile_issue<T>(W, SZ, base + (t + DP) * T, N, U, NG, uc, gsh, w[t % DP], sz[t % DP]);
    __builtin_amdgcn_sched_barrier(0);
    fold_rows<NR, T>(p, t * T, fl);
  }
  fold_finish<NR>(p);
  {
    float* rq = red + (wave * 4 + (lane >> 4)) * NR + fl.m;
    if ((lane & 15) < (NR < 16 ? NR : 16)) {
#pragma unroll
      for (int j = 0; j < (NR + 15) / 16; ++j) rq[16 * j] = p[16 * j];
    }
  }
  // the rows are finished by the row group's threads from LDS: across its waves a workgroup barrier; within a one-wave
  // group the wave's own LDS writes, ordered before its reads by a wavefront-scope fence (the other row groups of the
  // workgroup need not be waited for)
  if (nw > 1) {
    __syncthreads();
  } else {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  if constexpr (EPI == kOutRows) {
    if (tid < T * NT && base + tid < N) {
      y[base + tid] = (f16)row_total<NR>(red, gw0, nw, tid);
    }
  } else if constexpr (EPI == kOutRope) {
    if (tid < T * NT / 2 && 2 * rp + 1 < N) {
      const f16 a16 = (f16)row_total<NR>(red, gw0, nw, 2 * tid), b16 = (f16)row_total<NR>(red, gw0, nw, 2 * tid + 1);
      const int nq = in.rope.n_q, nkv = in.rope.n_kv, half = 1 << hb;
      f16 lo = a16, hi = b16;
      if (rvalid && rhead < nq + nkv) rope_rotate(a16, b16, rc, rs, lo, hi);
      f16* yh = y + ((size_t)rhead << in.rope.log2D);
      yh[ri] = rhead < nq ? lo : a16;
      yh[ri + half] = rhead < nq ? hi : b16;
      if (rvalid && rhead >= nq && rpage >= 0) {
        const bool is_k = rhead < nq + nkv;
        const int kvh = is_k ? rhead - nq : rhead - nq - nkv;
        const int slot = rpos & ((1 << in.rope.log2P) - 1);
        f16* dst = static_cast<f16*>(is_k ? in.rope.kc : in.rope.vc) +
                   (((((size_t)rpage * nkv + kvh) << in.rope.log2P) + slot) << in.rope.log2D);
        dst[ri] = lo;
        dst[ri + half] = hi;
      }
    }
  } else {
    if (tid < T * NT / 2 && base + 2 * tid + 1 < N) {
      const float g = row_total<NR>(red, gw0, nw, 2 * tid), up = row_total<NR>(red, gw0, nw, 2 * tid + 1);
      y[(base >> 1) + tid] = silu_mul((f16)g, (f16)up);
    }
  }
}

template <int R, int P>
void launch_rows(int waves, const void* packed, const void* sz, const void* x, void* y, int N, int K, int log2G,
                 hipStream_t st) {
  const int U = K >> 5;
  const int rows_per_block = R * waves;
  const int blocks = (N + rows_per_block - 1) / rows_per_block;
  // The transposed x layout pads the last step to 64 columns: ceil(U / 64) steps x 4 words x 64 lanes x 16 B.
  const size_t lds = (size_t)((U + 63) / 64) * 4 * 64 * 16;
  hipLaunchKernelGGL((gemv_w4a16_rows<R, P>), dim3(blocks), dim3(64 * waves), lds, st,
                     (const u32x4*)packed, (const uint32_t*)sz, (const u32x4*)x, (f16*)y, N, U, log2G - 5);
}

template <int R>
void launch_rows_p(int waves, int pf, const void* packed, const void* sz, const void* x, void* y, int N, int K,
                   int log2G, hipStream_t st) {
  // prefetch depth 2^pf column steps, capped so that at most 16 loads of 16 B per lane are in flight (R * depth <= 16)
  const int P = min(1 << pf, 16 / R);
  if constexpr (R <= 2) {
    if (P >= 8) return launch_rows<R, 8>(waves, packed, sz, x, y, N, K, log2G, st);
  }
  if constexpr (R <= 4) {
    if (P >= 4) return launch_rows<R, 4>(waves, packed, sz, x, y, N, K, log2G, st);
  }
  if (P >= 2) return launch_rows<R, 2>(waves, packed, sz, x, y, N, K, log2G, st);
  launch_rows<R, 1>(waves, packed, sz, x, y, N, K, log2G, st);
}

// warps: waves per workgroup, 0 or a multiple of ceil(K / 2048) up to 16 (checked by the C ABI): that many / ceil(K /
// 2048) row groups per workgroup (0 = one).
template <int T, int NT, int PRO, int EPI>
void launch_tile_nt(int warps, const void* packed, const void* sz, const GemvInput& in, void* y, int N, int K,
                    int log2G, hipStream_t st) {
  if constexpr (EPI != kOutRows && (T * NT) % 2 != 0) {
    return;  // rejected by the host checks (R * 2^pf >= 2); never instantiated as a kernel
  } else {
    const int U = K >> 5;
    const int nw = (U + 63) / 64;
    const int groups = warps > 0 ? warps / nw : 1;
    const int rows = T * NT * groups;
    hipLaunchKernelGGL((gemv_w4a16_tile<T, NT, PRO, EPI>), dim3((N + rows - 1) / rows), dim3(64 * nw * groups), 0,
                       st, (const u32x4*)packed, (const uint32_t*)sz,
                       is_combine(PRO) ? static_cast<const void*>(in.comb.o_part) : in.x, N, U, log2G - 5, groups,
                       is_combine(PRO) ? static_cast<const void*>(in.comb.m_part) : in.norm_w,
                       is_combine(PRO) ? static_cast<const void*>(in.comb.l_part) : in.delta, (f16*)y, in);
  }
}

template <int T, int PRO, int EPI>
void launch_tile(int warps, int pf, const void* packed, const void* sz, const GemvInput& in, void* y, int N, int K,
                 int log2G, hipStream_t st) {
  switch (pf) {
    case 0: launch_tile_nt<T, 1, PRO, EPI>(warps, packed, sz, in, y, N, K, log2G, st); break;
    case 1: launch_tile_nt<T, 2, PRO, EPI>(warps, packed, sz, in, y, N, K, log2G, st); break;
    case 2: launch_tile_nt<T, 4, PRO, EPI>(warps, packed, sz, in, y, N, K, log2G, st); break;
    default: launch_tile_nt<T, 8, PRO, EPI>(warps, packed, sz, in, y, N, K, log2G, st); break;
  }
}

template <int PRO, int EPI = kOutRows>
void launch_tile_r(int R, int warps, int pf, const void* packed, const void* sz, const GemvInput& in, void* y, int N,
                   int K, int log2G, hipStream_t st) {
  switch (R) {
    case 1: launch_tile<1, PRO, EPI>(warps, pf, packed, sz, in, y, N, K, log2G, st); break;
    case 2: launch_tile<2, PRO, EPI>(warps, pf, packed, sz, in, y, N, K, log2G, st); break;
    case 4: launch_tile<4, PRO, EPI>(warps, pf, packed, sz, in, y, N, K, log2G, st); break;
    default: launch_tile<8, PRO, EPI>(warps, pf, packed, sz, in, y, N, K, log2G, st); break;
  }
}

template <int R>
void launch_splitk(int waves, int pf, const void* packed, const void* sz, const void* x, void* y, int N, int K,
                   int log2G, hipStream_t st) {
  const int U = K >> 5;
  const int blocks = (N + R - 1) / R;
  const int gsh = log2G - 5;
  if (pf)
    hipLaunchKernelGGL((gemv_w4a16_splitk<R, true>), dim3(blocks), dim3(64 * waves), 0, st, (const u32x4*)packed,
                       (const uint32_t*)sz, (const u32x4*)x, (f16*)y, N, U, gsh);
  else
    hipLaunchKernelGGL((gemv_w4a16_splitk<R, false>), dim3(blocks), dim3(64 * waves), 0, st, (const u32x4*)packed,
                       (const uint32_t*)sz, (const u32x4*)x, (f16*)y, N, U, gsh);
}

}  // namespace

void gemv_default_config(int N, int K, int* stage, int* R, int* waves, int* pf) {
  // Row tiles of 2 rows, one tile per workgroup, while the workgroup can cover K (K <= 32768); split-K beyond.
  (void)N;
  if (K <= kGemvRowsMaxK) {
    *stage = 4;
    *R = 2;
    *waves = 0;
    *pf = 0;
    return;
  }
  *stage = 3;
  *R = 2;
  *waves = 16;
  *pf = 1;
}

void launch_gemv_w4a16(int stage, int R, int waves, int pf, const void* packed, const void* sz, const void* x,
                       void* y, int N, int K, int log2G, hipStream_t st) {
  if (stage == 0) {
    const int wpb = waves > 0 ? waves : 4;
    hipLaunchKernelGGL(gemv_w4a16_exact, dim3((N + wpb - 1) / wpb), dim3(64 * wpb), 0, st, (const uint32_t*)packed,
                       (const uint32_t*)sz, (const f16*)x, (f16*)y, N, K, log2G);
    return;
  }
  if (stage == 4) {
    GemvInput in{};
    in.x = x;
    launch_tile_r<kInPlain>(R, waves, pf, packed, sz, in, y, N, K, log2G, st);
    return;
  }
  if (waves <= 0) waves = stage == 3 ? min(16, ((K >> 5) + 63) / 64) : 4;
  if (stage == 1) R = 1;
  if (stage == 1 || stage == 2) {
    switch (R) {
      case 1: launch_rows_p<1>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
      case 2: launch_rows_p<2>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
      case 4: launch_rows_p<4>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
      default: launch_rows_p<8>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    }
    return;
  }
  switch (R) {
    case 1: launch_splitk<1>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    case 2: launch_splitk<2>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    case 4: launch_splitk<4>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
    default: launch_splitk<8>(waves, pf, packed, sz, x, y, N, K, log2G, st); break;
  }
}

void launch_gemv_w4a16_fused(int prologue, int epilogue, int R, int warps, int pf, const void* packed, const void* sz,
                             const GemvInput& in, void* y, int N, int K, int log2G, hipStream_t st) {
  if (epilogue == kOutSwiglu) {
    if (prologue == kInRmsNorm)
      launch_tile_r<kInRmsNorm, kOutSwiglu>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    else
      launch_tile_r<kInPlain, kOutSwiglu>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    return;
  }
  if (epilogue == kOutRope) {
    if (prologue == kInRmsNorm)
      launch_tile_r<kInRmsNorm, kOutRope>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    else
      launch_tile_r<kInPlain, kOutRope>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    return;
  }
  if (prologue == 2) {
    const int ms = in.comb.max_splits;
    if (ms <= 4)
      launch_tile_r<kInCombine4>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    else if (ms <= 8)
      launch_tile_r<kInCombine8>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    else
      launch_tile_r<kInCombine16>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
    return;
  }
  launch_tile_r<kInRmsNorm>(R, warps, pf, packed, sz, in, y, N, K, log2G, st);
}

}  // namespace dk
