// fp16-weight GEMV for batch-1 decode on gfx950:  y[N] = W[N, K] . x[K]   (fp16 in/out, fp32 accumulation)
//
// The LM head of an INT4 model keeps fp16 weights; the reference runs it as torch.mm(x, W^T) on cuBLAS
// (runtime/model.py:187). At TinyLlama shape it is 32000 x 2048 = 131 MB, a fifth of a token's bytes, so it is an HBM
// stream like the INT4 GEMV and gets its own kernel, optionally with the final residual + RMSNorm in front
// (kernels/fused_norm.cu:8-54 rounding points) so the step's last add_rmsnorm launch disappears.
//
// Layout: W row-major fp16 [N, K] (the HF lm_head.weight as stored), 16-byte chunks of 8 weights; U = K / 8 chunks
// per row. Every wave owns whole rows: lane l holds chunks l, l + 64, ..., l + 64 (C - 1) of x in registers
// (C = ceil(U / 64)), so one wave covers K alone and a row's sum is one DPP reduction, with no LDS and no barrier.
// A wave walks NT tiles of T consecutive rows; each tile is T x C 16-byte loads per lane (T x C x 1 KB per wave, every
// wave load 1 KB contiguous), and the loads of tile t + 1 are issued before tile t is computed (double buffering,
// pinned by scheduling barriers). Products are v_dot2_f32_f16 (exact fp16 x fp16 products, fp32 sums).
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

template <int C, int T>
__device__ __forceinline__ void f16_issue(const u32x4* __restrict__ W, int row0, int N, int U, int lane,
                                          u32x4 (&w)[T][C]) {
#pragma unroll
  for (int r = 0; r < T; ++r) {
    const size_t rb = (size_t)min(row0 + r, N - 1) * U;
#pragma unroll
    for (int c = 0; c < C; ++c) w[r][c] = load_stream(W + rb + min(lane + 64 * c, U - 1));
  }
}

template <int C, int T>
__device__ __forceinline__ void f16_rows(const u32x4 (&w)[T][C], const u32x4 (&xc)[C], int lane, int U,
                                         float (&v)[T]) {
#pragma unroll
  for (int r = 0; r < T; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      float p = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) p = dot2(as_f16x2(w[r][c][e]), as_f16x2(xc[c][e]), p);
      acc += lane + 64 * c < U ? p : 0.f;  // dead chunks (past K) contribute 0 whatever the clamped load held
    }
    v[r] = wave_sum_lane63(acc);
  }
}

// x operand per lane: chunk ci = lane + 64 c of
//   PRO 0  x
//   PRO 1  add_rmsnorm(x, delta, norm_w): xn = fp16(x + delta), r = 1 / sqrt(sum(xn^2) / K + eps) over the whole
//          vector (one wave sum), value = norm_w * fp16(float(xn) * r). Wave 0 of workgroup 0 writes xn to x_out.
// f16_input_load issues the operand loads before any weight load of the wave (a wave's vector loads return in issue
// order, so operand loads queued behind the weight stream would hold back the prologue); f16_input_finish computes
// the operand once they have arrived.
template <int C, int PRO>
__device__ __forceinline__ void f16_input_load(const void* x, const void* norm_w, const void* delta, int lane, int U,
                                               u32x4 (&xr)[C], u32x4 (&dr)[C], u32x4 (&wn)[C]) {
  const u32x4* X = reinterpret_cast<const u32x4*>(x);
#pragma unroll
  for (int c = 0; c < C; ++c) xr[c] = X[min(lane + 64 * c, U - 1)];
  if constexpr (PRO == 1) {
    const u32x4* Wn = reinterpret_cast<const u32x4*>(norm_w);
#pragma unroll
    for (int c = 0; c < C; ++c) wn[c] = Wn[min(lane + 64 * c, U - 1)];
    if (delta != nullptr) {
      const u32x4* Dl = reinterpret_cast<const u32x4*>(delta);
#pragma unroll
      for (int c = 0; c < C; ++c) dr[c] = Dl[min(lane + 64 * c, U - 1)];
    }
  }
}

template <int C, int PRO>
__device__ __forceinline__ void f16_input_finish(const GemvInput& in, const void* delta, int lane, int U, bool writer,
                                                 u32x4 (&xc)[C], const u32x4 (&dr)[C], const u32x4 (&wn)[C]) {
  if constexpr (PRO == 0) {
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (lane + 64 * c >= U) xc[c] = u32x4{0u, 0u, 0u, 0u};
  } else {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ci = lane + 64 * c;
      const bool live = ci < U;
      if (delta != nullptr) {
#pragma unroll
        for (int e = 0; e < 4; ++e) xc[c][e] = as_u32(as_f16x2(xc[c][e]) + as_f16x2(dr[c][e]));
      }
      if (!live) xc[c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(xc[c][e]);
        const float a = (float)h.x, b = (float)h.y;
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
      if (writer && live && in.x_out != nullptr) reinterpret_cast<u32x4*>(in.x_out)[ci] = xc[c];
    }
    const float r = 1.0f / sqrtf(wave_sum_all(ss) / (float)(U << 3) + in.eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(xc[c][e]);
        const f16x2 hn = {(f16)((float)h.x * r), (f16)((float)h.y * r)};
        xc[c][e] = as_u32(as_f16x2(wn[c][e]) * hn);
      }
    }
  }
}

// Pipeline: operand loads, the weight loads of tiles 0 and 1, the operand, then per tile: compute it from its buffer
// and refill that buffer with tile t + 2.
template <int C, int T, int NT, int PRO>
// The arguments the first loads need come first (preloaded into scalar registers at launch).
__global__ void __launch_bounds__(512)
gemv_f16_rows(const u32x4* __restrict__ W, const void* X, int N, int U, const void* norm_w, const void* delta,
              f16* __restrict__ y, const GemvInput in) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * (T * NT);
  if (row0 >= N) return;  // whole wave past the last row (no barrier follows)
  u32x4 xc[C], dr[C], wn[C];
  f16_input_load<C, PRO>(X, norm_w, delta, lane, U, xc, dr, wn);
  u32x4 w[2][T][C];
  f16_issue<C, T>(W, row0, N, U, lane, w[0]);
  if constexpr (NT > 1) f16_issue<C, T>(W, row0 + T, N, U, lane, w[1]);
  __builtin_amdgcn_sched_barrier(0);
  f16_input_finish<C, PRO>(in, delta, lane, U, blockIdx.x == 0 && wave == 0, xc, dr, wn);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float v[T];
    f16_rows<C, T>(w[t & 1], xc, lane, U, v);
    if (t + 2 < NT) f16_issue<C, T>(W, row0 + (t + 2) * T, N, U, lane, w[t & 1]);
    __builtin_amdgcn_sched_barrier(0);
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < T; ++r)
        if (row0 + t * T + r < N) y[row0 + t * T + r] = (f16)v[r];
    }
  }
}

template <int C, int T, int NT, int PRO>
void launch_f16_nt(int waves, const void* w, const GemvInput& in, void* y, int N, int K, hipStream_t st) {
  if constexpr (T * C > kGemvF16MaxLoads) {
    return;  // rejected by the host checks (two buffers of T x C chunks must fit the register file)
  } else {
    const int rows_per_block = waves * T * NT;
    hipLaunchKernelGGL((gemv_f16_rows<C, T, NT, PRO>), dim3((N + rows_per_block - 1) / rows_per_block),
                       dim3(64 * waves), 0, st, (const u32x4*)w, in.x, N, K >> 3, in.norm_w, in.delta, (f16*)y, in);
  }
}

template <int C, int T, int PRO>
void launch_f16_t(int waves, int pf, const void* w, const GemvInput& in, void* y, int N, int K, hipStream_t st) {
  switch (pf) {
    case 0: launch_f16_nt<C, T, 1, PRO>(waves, w, in, y, N, K, st); break;
    case 1: launch_f16_nt<C, T, 2, PRO>(waves, w, in, y, N, K, st); break;
    case 2: launch_f16_nt<C, T, 4, PRO>(waves, w, in, y, N, K, st); break;
    default: launch_f16_nt<C, T, 8, PRO>(waves, w, in, y, N, K, st); break;
  }
}

template <int C, int PRO>
void launch_f16_c(int R, int waves, int pf, const void* w, const GemvInput& in, void* y, int N, int K,
                  hipStream_t st) {
  switch (R) {
    case 1: launch_f16_t<C, 1, PRO>(waves, pf, w, in, y, N, K, st); break;
    case 2: launch_f16_t<C, 2, PRO>(waves, pf, w, in, y, N, K, st); break;
    default: launch_f16_t<C, 4, PRO>(waves, pf, w, in, y, N, K, st); break;
  }
}

template <int PRO>
void launch_f16(int R, int waves, int pf, const void* w, const GemvInput& in, void* y, int N, int K,
                hipStream_t st) {
  const int chunks = ((K >> 3) + 63) / 64;
  if (chunks <= 1) return launch_f16_c<1, PRO>(R, waves, pf, w, in, y, N, K, st);
  if (chunks <= 2) return launch_f16_c<2, PRO>(R, waves, pf, w, in, y, N, K, st);
  if (chunks <= 4) return launch_f16_c<4, PRO>(R, waves, pf, w, in, y, N, K, st);
  launch_f16_c<8, PRO>(R, waves, pf, w, in, y, N, K, st);
}

}  // namespace

void launch_gemv_f16(int prologue, int R, int waves, int pf, const void* w, const GemvInput& in, void* y, int N,
                     int K, hipStream_t st) {
  if (waves == 0) waves = 4;
  if (prologue == 1)
    launch_f16<1>(R, waves, pf, w, in, y, N, K, st);
  else
    launch_f16<0>(R, waves, pf, w, in, y, N, K, st);
}

}  // namespace dk
