// Single-pass bandwidth kernels of the decode step on gfx950: fused residual + RMSNorm, fused SwiGLU, RoPE + paged
// KV append. Each rounds to fp16 at exactly the points the reference's fp16 semantics do (reference/ref_ops.py).
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

// ---------------------------------------------------------------------------------------------------------------
// Residual + RMSNorm of one row per workgroup, the row held in registers (dk_add_rmsnorm is the one-row case, in
// place; dk_rmsnorm_rows the prefill rows, with an optional gather):
//   xn = fp16(x_in[src] + delta[r])   (delta optional; src = rows[r] with a gather index, else r)
//   x_out[r] = xn,  out[r] = w * fp16(float(xn) * rr),  rr = 1 / sqrt(sum(float(xn)^2) / H + eps)
// with the reference's rounding points (reference/ref_ops.py:15-20). Thread t of T owns the C 16-byte chunks t, t + T,
// ..., t + (C - 1) T. Every operand load -- the row, the delta and the norm weight, which is needed only after the
// reduction -- is issued unconditionally before any arithmetic (chunk indices clamped; a missing delta re-reads the
// row), so the weight's latency hides behind the sum and the row is never read back. One wave sum per wave, one LDS
// exchange. x_out may be x_in itself when there is no gather: a thread writes only chunks it has already read.
// A gathered row index outside [0, n_src) reads row 0 and poisons the row with NaN instead of reading out of bounds.
// PARTS: the delta is the split-K GEMM's fp32 partials, parts[s * pstride + r * H + n] for s < splits, rounded to fp16
// after summing them in split order exactly as gemm_splitk_reduce does (the GEMM's reduce launch folded in here; loads
// of up to four splits in flight together).
template <int C, bool PARTS = false>
__global__ void __launch_bounds__(1024)
row_norm_kernel(const f16* x_in, const int64_t* __restrict__ rows, int n_src, const f16* __restrict__ delta,
                const f16* __restrict__ w, f16* x_out, f16* __restrict__ out, int H, float eps,
                const float* __restrict__ parts, int splits, long long pstride) {
  __shared__ float part[16];
  const int r = blockIdx.x, tid = threadIdx.x, T = blockDim.x, U = H >> 3;
  const long long sr = rows != nullptr ? rows[r] : r;
  const bool bad = sr < 0 || sr >= n_src;
  const u32x4* src = reinterpret_cast<const u32x4*>(x_in + (size_t)(bad ? 0 : sr) * H);
  const u32x4* dl = delta != nullptr ? reinterpret_cast<const u32x4*>(delta + (size_t)r * H) : src;
  const u32x4* wc = reinterpret_cast<const u32x4*>(w);
  u32x4 xv[C], dv[C], wv[C];
#pragma unroll
  for (int c = 0; c < C; ++c) xv[c] = src[min(tid + c * T, U - 1)];
  if constexpr (PARTS) {
    const float4* pr = reinterpret_cast<const float4*>(parts + (size_t)r * H);
    float4 lo[C], hi[C];  // running sums of the chunk's 8 values, split 0 first
    for (int s0 = 0; s0 < splits; s0 += 4) {
      float4 bl[C][4], bh[C][4];
#pragma unroll
      for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4* ps = pr + (size_t)min(s0 + k, splits - 1) * (size_t)(pstride >> 2) + 2 * min(tid + c * T, U - 1);
          bl[c][k] = ps[0];
          bh[c][k] = ps[1];
        }
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (s0 + k >= splits) continue;
          if (s0 + k == 0) {
            lo[c] = bl[c][k];
            hi[c] = bh[c][k];
          } else {
            lo[c].x += bl[c][k].x; lo[c].y += bl[c][k].y; lo[c].z += bl[c][k].z; lo[c].w += bl[c][k].w;
            hi[c].x += bh[c][k].x; hi[c].y += bh[c][k].y; hi[c].z += bh[c][k].z; hi[c].w += bh[c][k].w;
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c)
      dv[c] = u32x4{as_u32(f16x2{(f16)lo[c].x, (f16)lo[c].y}), as_u32(f16x2{(f16)lo[c].z, (f16)lo[c].w}),
                    as_u32(f16x2{(f16)hi[c].x, (f16)hi[c].y}), as_u32(f16x2{(f16)hi[c].z, (f16)hi[c].w})};
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) dv[c] = dl[min(tid + c * T, U - 1)];
  }
#pragma unroll
  for (int c = 0; c < C; ++c) wv[c] = wc[min(tid + c * T, U - 1)];
  u32x4* xo = reinterpret_cast<u32x4*>(x_out + (size_t)r * H);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int u = tid + c * T;
    if (PARTS || delta != nullptr) {
#pragma unroll
      for (int k = 0; k < 4; ++k) xv[c][k] = as_u32(as_f16x2(xv[c][k]) + as_f16x2(dv[c][k]));
    }
    if (bad) xv[c] = u32x4{0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};  // fp16 NaN
    if (u < U) {
      xo[u] = xv[c];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const f16x2 h = as_f16x2(xv[c][k]);
        const float a = (float)h.x, b = (float)h.y;
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
  ss = group_sum<kWave>(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (T >> 6); ++i) tot += part[i];
  const float rr = bad ? __builtin_nanf("") : 1.0f / sqrtf(tot / (float)H + eps);
  u32x4* o = reinterpret_cast<u32x4*>(out + (size_t)r * H);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int u = tid + c * T;
    if (u >= U) continue;
    u32x4 ov;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f16x2 h = as_f16x2(xv[c][k]);
      const f16x2 hn = {(f16)((float)h.x * rr), (f16)((float)h.y * rr)};
      ov[k] = as_u32(as_f16x2(wv[c][k]) * hn);
    }
    o[u] = ov;
  }
}

// Residual + RMSNorm of one row too long for registers (H > kRowNormMaxH; the reference's add_rmsnorm takes any
// H % 8 == 0, kernels/bindings.cpp:64-72): the same arithmetic in two passes over the row in memory. Pass 1 adds the
// delta, writes xn to x (in place) and sums the squares; pass 2 re-reads the chunks this thread wrote and writes
// out = w * fp16(float(xn) * rr). One workgroup; thread t owns chunks t, t + T, ...
__global__ void __launch_bounds__(1024)
row_norm_long_kernel(f16* x, const f16* __restrict__ delta, const f16* __restrict__ w, f16* __restrict__ out, int H,
                     float eps) {
  __shared__ float part[16];
  const int tid = threadIdx.x, T = blockDim.x, U = H >> 3;
  u32x4* xc = reinterpret_cast<u32x4*>(x);
  const u32x4* dl = reinterpret_cast<const u32x4*>(delta);
  float ss = 0.f;
  for (int u = tid; u < U; u += T) {
    u32x4 xv = xc[u];
    if (delta != nullptr) {
      const u32x4 dv = dl[u];
#pragma unroll
      for (int k = 0; k < 4; ++k) xv[k] = as_u32(as_f16x2(xv[k]) + as_f16x2(dv[k]));
      xc[u] = xv;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f16x2 h = as_f16x2(xv[k]);
      const float a = (float)h.x, b = (float)h.y;
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = group_sum<kWave>(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (T >> 6); ++i) tot += part[i];
  const float rr = 1.0f / sqrtf(tot / (float)H + eps);
  const u32x4* wc = reinterpret_cast<const u32x4*>(w);
  u32x4* o = reinterpret_cast<u32x4*>(out);
  for (int u = tid; u < U; u += T) {
    const u32x4 xv = xc[u], wv = wc[u];
    u32x4 ov;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f16x2 h = as_f16x2(xv[k]);
      const f16x2 hn = {(f16)((float)h.x * rr), (f16)((float)h.y * rr)};
      ov[k] = as_u32(as_f16x2(wv[k]) * hn);
    }
    o[u] = ov;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// out[i] = fp16(silu(float(gate[i]))) * up[i] in fp16, gate = gu[0:I], up = gu[I:2I]   (reference/ref_ops.py:23-27).
__global__ void __launch_bounds__(256)
swiglu_kernel(const f16* __restrict__ gu, f16* __restrict__ out, int I) {
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= I) return;
  const u32x4 gv = *reinterpret_cast<const u32x4*>(gu + i);
  const u32x4 uv = *reinterpret_cast<const u32x4*>(gu + I + i);
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f16x2 g2 = as_f16x2(gv[k]), u2 = as_f16x2(uv[k]);
    const f16x2 r = {silu_mul(g2.x, u2.x), silu_mul(g2.y, u2.y)};
    o[k] = as_u32(r);
  }
  *reinterpret_cast<u32x4*>(out + i) = o;
}

// ---------------------------------------------------------------------------------------------------------------
// RoPE, rotate_half pairs (i, i + D/2), at position *pos, then paged K/V append   (reference/ref_ops.py:36-53).
// One thread per (head, pair): q heads rotate in place, k heads rotate into the cache, v heads copy into the cache.
// fp32 products are rounded separately (no contraction), exactly as the reference's elementwise fp32 ops, so the
// rotated values are bit-identical to the reference's.
template <int D>
__global__ void __launch_bounds__(256)
rope_append_kernel(f16* __restrict__ qkv, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                   const int32_t* __restrict__ pos_ptr, const int32_t* __restrict__ bt, f16* __restrict__ kc,
                   f16* __restrict__ vc, int n_q, int n_kv, int log2P, int max_pos, int n_pages, int n_bt,
                   int row_stride) {
#pragma clang fp contract(off)
  constexpr int HALF = D / 2;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int head = idx / HALF, i = idx % HALF;
  if (head >= n_q + 2 * n_kv) return;
  // row y of a batch of tokens (prefill) sits at position *pos + y; the decode op has one row
  const int pos = *pos_ptr + (int)blockIdx.y;
  qkv += (size_t)blockIdx.y * row_stride;
  if (pos < 0 || pos >= max_pos) return;
  const int lp = pos >> log2P;
  int page = -1;
  if (lp < n_bt) {
    page = bt[lp];
    if (page < 0 || page >= n_pages) page = -1;
  }
  const int slot = pos & ((1 << log2P) - 1);
  f16* xh = qkv + (size_t)head * D;
  if (head < n_q + n_kv) {
    const float c = cos_t[(size_t)pos * HALF + i], s = sin_t[(size_t)pos * HALF + i];
    const float a = (float)xh[i], b = (float)xh[i + HALF];
    const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    const f16 lo = (f16)(ac - bs), hi = (f16)(bc + as);
    if (head < n_q) {
      xh[i] = lo;
      xh[i + HALF] = hi;
    } else if (page >= 0) {
      f16* dst = kc + ((((size_t)page * n_kv + (head - n_q)) << log2P) + slot) * D;
      dst[i] = lo;
      dst[i + HALF] = hi;
    }
  } else if (page >= 0) {
    f16* dst = vc + ((((size_t)page * n_kv + (head - n_q - n_kv)) << log2P) + slot) * D;
    dst[i] = xh[i];
    dst[i + HALF] = xh[i + HALF];
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Greedy token pick closing the decode step: tok = argmax(logits) (lowest index among equal maxima, NaN counts as
// largest like torch.argmax), then *pos += 1 when pos is given (runtime/model.py:232-233 of the reference as one
// launch). One workgroup of 1024 threads: each thread issues all of its 16-byte chunks of a batch (kArgmaxBatch per
// thread) before comparing, so the whole vector is in flight at once instead of one 2-byte load per step; a scalar
// head and tail cover a logits pointer that is not 16-byte aligned and V % 8.
constexpr int kArgmaxBatch = 4;

__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

__device__ __forceinline__ void take(float v, int i, float& bv, int& bi) {
  if (better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

__global__ void __launch_bounds__(1024)
argmax_advance_kernel(const f16* __restrict__ logits, int V, int64_t* __restrict__ tok, int32_t* __restrict__ pos) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int tid = threadIdx.x, nt = blockDim.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // elements [0, h) before the first 16-byte boundary, chunks of 8 over [h, h + 8 * nc), scalar tail after
  const int h = min(V, (int)(((16u - ((uint32_t)(uintptr_t)logits & 15u)) & 15u) >> 1));
  const int nc = (V - h) >> 3;
  if (tid < h) take((float)logits[tid], tid, bv, bi);
  const u32x4* C = reinterpret_cast<const u32x4*>(logits + h);
  for (int c0 = tid; c0 < nc; c0 += kArgmaxBatch * nt) {
    u32x4 v[kArgmaxBatch];
#pragma unroll
    for (int b = 0; b < kArgmaxBatch; ++b) {
      const int c = c0 + b * nt;
      v[b] = c < nc ? C[c] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int b = 0; b < kArgmaxBatch; ++b) {
      const int c = c0 + b * nt;
      if (c < nc) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 p = as_f16x2(v[b][e]);
          const int i = h + 8 * c + 2 * e;
          take((float)p.x, i, bv, bi);
          take((float)p.y, i + 1, bv, bi);
        }
      }
    }
  }
  const int t0 = h + 8 * nc;
  if (t0 + tid < V) take((float)logits[t0 + tid], t0 + tid, bv, bi);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    take(ov, oi, bv, bi);
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < (nt >> 6); ++w) take(sv[w], si[w], bv, bi);
    tok[0] = (int64_t)bi;
    if (pos != nullptr) pos[0] += 1;
  }
}

// The same pick over many workgroups (for large V, where one workgroup's compare work dominates: 128256 logits cost a
// single CU about 20 us). Every element maps to a 64-bit key that orders as argmax ranks:
//   high word: 0xFFFFFFFF for NaN, else the float's bits made monotonic (negatives inverted, positives with the sign
//              bit set; -0 first turned into +0 so that the two zeros tie as they compare equal);
//   low word:  ~index, so that among equal values the lowest index has the largest key.
// Workgroup w takes the 16-byte chunks [w * kArgmaxWgChunks, (w + 1) * kArgmaxWgChunks), workgroup 0 also the unaligned
// head and the tail. Each workgroup folds its best key into work[0] with a device-scope atomic max, then counts itself
// in work[1] with a device-scope release / acquire atomic add; the workgroup that reads n - 1 arrives last, and every
// other maximum happens before its load of work[0]: it writes *tok and *pos + 1, and resets work[0] and work[1] to 0
// for the next call. No workgroup waits for another.
constexpr int kArgmaxWgThreads = 256;
constexpr int kArgmaxWgChunks = 2 * kArgmaxWgThreads;  // two 16-byte chunks (16 logits) per thread

__global__ void __launch_bounds__(kArgmaxWgThreads)
argmax_split_kernel(const f16* __restrict__ logits, int V, int h, int nc, int64_t* __restrict__ tok,
                    int32_t* __restrict__ pos, unsigned long long* __restrict__ work) {
  __shared__ unsigned long long s_k[kArgmaxWgThreads / 64];
  const int tid = threadIdx.x;
  unsigned long long best = 0;  // below every key (the smallest key, -inf at index 2^32 - 1, is still above 0)
  const u32x4* C = reinterpret_cast<const u32x4*>(logits + h);
  const int c0 = blockIdx.x * kArgmaxWgChunks + tid;
  u32x4 v[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) v[b] = c0 + b * kArgmaxWgThreads < nc ? C[c0 + b * kArgmaxWgThreads] : u32x4{0u, 0u, 0u, 0u};
  if (blockIdx.x == 0) {
    if (tid < h) best = max(best, (unsigned long long)argmax_key((float)logits[tid], tid));
    const int t0 = h + 8 * nc;
    if (t0 + tid < V) best = max(best, (unsigned long long)argmax_key((float)logits[t0 + tid], t0 + tid));
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int c = c0 + b * kArgmaxWgThreads;
    if (c < nc) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 p = as_f16x2(v[b][e]);
        const int i = h + 8 * c + 2 * e;
        best = max(best, (unsigned long long)argmax_key((float)p.x, i));
        best = max(best, (unsigned long long)argmax_key((float)p.y, i + 1));
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) best = max(best, (unsigned long long)__shfl_xor(best, o, kWave));
  if ((tid & 63) == 0) s_k[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxWgThreads / 64; ++w) best = max(best, s_k[w]);
    // The arrival is a release / acquire RMW at device scope: this workgroup's maximum (sequenced before its arrival)
    // happens before the last arrival's load of work[0], because the last arrival's acquire reads the end of the
    // counter's release sequence, which holds every earlier arrival.
    __hip_atomic_fetch_max(&work[0], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long prev =
        __hip_atomic_fetch_add(&work[1], 1ull, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (unsigned long long)(gridDim.x - 1)) {
      const unsigned long long k = __hip_atomic_load(&work[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      tok[0] = (int64_t)(uint32_t)~(uint32_t)k;
      if (pos != nullptr) pos[0] += 1;
      __hip_atomic_store(&work[0], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&work[1], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

// Chunks per thread: the smallest C in {1, 2, 4, 8} with 1024 C 16-byte chunks covering the row (H <= kRowNormMaxH).
static void launch_row_norm(const void* x_in, const int64_t* rows, int n_src, const void* delta, const void* w,
                            void* x_out, void* out, int M, int H, float eps, hipStream_t st) {
  const int U = H >> 3;
  int C = 1;
  while (C < 8 && C * 1024 < U) C *= 2;
  const int T = min(1024, ((U + C - 1) / C + 63) / 64 * 64);
  const f16 *xi = (const f16*)x_in, *d = (const f16*)delta, *wn = (const f16*)w;
  f16 *xo = (f16*)x_out, *o = (f16*)out;
  auto kernel = C == 1 ? row_norm_kernel<1> : C == 2 ? row_norm_kernel<2> : C == 4 ? row_norm_kernel<4>
                                                                            : row_norm_kernel<8>;
  hipLaunchKernelGGL(kernel, dim3(M), dim3(T), 0, st, xi, rows, n_src, d, wn, xo, o, H, eps, (const float*)nullptr, 0,
                     0LL);
}

void launch_add_rmsnorm(void* x, const void* delta, const void* w, void* out, int H, float eps, hipStream_t st) {
  if (H > kRowNormMaxH) {
    hipLaunchKernelGGL(row_norm_long_kernel, dim3(1), dim3(1024), 0, st, (f16*)x, (const f16*)delta, (const f16*)w,
                       (f16*)out, H, eps);
    return;
  }
  launch_row_norm(x, nullptr, 1, delta, w, x, out, 1, H, eps, st);
}

void launch_swiglu(const void* gu, void* out, int I, hipStream_t st) {
  const int n = I / 8;
  const int threads = 256;
  hipLaunchKernelGGL(swiglu_kernel, dim3((n + threads - 1) / threads), dim3(threads), 0, st, (const f16*)gu,
                     (f16*)out, I);
}

void launch_rope_append(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                        void* kc, void* vc, int n_q, int n_kv, int head_dim, int log2P, int max_pos, int n_pages,
                        int n_bt, int rows, hipStream_t st) {
  const int pairs = (n_q + 2 * n_kv) * (head_dim / 2);
  const int threads = 256;
  const dim3 grid((pairs + threads - 1) / threads, rows);
  const int stride = (n_q + 2 * n_kv) * head_dim;
  if (head_dim == 64)
    hipLaunchKernelGGL((rope_append_kernel<64>), grid, dim3(threads), 0, st, (f16*)qkv, cos_t, sin_t, pos, bt,
                       (f16*)kc, (f16*)vc, n_q, n_kv, log2P, max_pos, n_pages, n_bt, stride);
  else
    hipLaunchKernelGGL((rope_append_kernel<128>), grid, dim3(threads), 0, st, (f16*)qkv, cos_t, sin_t, pos, bt,
                       (f16*)kc, (f16*)vc, n_q, n_kv, log2P, max_pos, n_pages, n_bt, stride);
}

void launch_rmsnorm_rows(const void* x_in, const int64_t* rows, int n_src, const void* delta, const void* w, void* x_out,
                         void* out, int M, int H, float eps, hipStream_t st) {
  launch_row_norm(x_in, rows, n_src, delta, w, x_out, out, M, H, eps, st);
}

void launch_rmsnorm_rows_parts(const void* x_in, const float* parts, int splits, long long pstride, const void* w,
                               void* x_out, void* out, int M, int H, float eps, hipStream_t st) {
  const int U = H >> 3;
  int C = 1;
  while (C < 8 && C * 1024 < U) C *= 2;
  const int T = min(1024, ((U + C - 1) / C + 63) / 64 * 64);
  auto kernel = C == 1 ? row_norm_kernel<1, true> : C == 2 ? row_norm_kernel<2, true>
                : C == 4 ? row_norm_kernel<4, true> : row_norm_kernel<8, true>;
  hipLaunchKernelGGL(kernel, dim3(M), dim3(T), 0, st, (const f16*)x_in, nullptr, M, nullptr, (const f16*)w,
                     (f16*)x_out, (f16*)out, H, eps, parts, splits, pstride);
}

void launch_argmax_advance(const void* logits, int V, int64_t* tok, int32_t* pos, hipStream_t st) {
  hipLaunchKernelGGL(argmax_advance_kernel, dim3(1), dim3(1024), 0, st, (const f16*)logits, V, tok, pos);
}

void launch_argmax_split(const void* logits, int V, int64_t* tok, int32_t* pos, unsigned long long* work,
                         hipStream_t st) {
  const int h = min(V, (int)(((16u - ((uint32_t)(uintptr_t)logits & 15u)) & 15u) >> 1));
  const int nc = (V - h) >> 3;
  const int blocks = max(1, (nc + kArgmaxWgChunks - 1) / kArgmaxWgChunks);
  hipLaunchKernelGGL(argmax_split_kernel, dim3(blocks), dim3(kArgmaxWgThreads), 0, st, (const f16*)logits, V, h, nc,
                     tok, pos, work);
}

}  // namespace dk
