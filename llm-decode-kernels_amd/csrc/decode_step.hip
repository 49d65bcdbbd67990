// Persistent batch-1 decode step on gfx950: one launch runs every layer, the LM head and the argmax of
// runtime/model.py:216-233 (the reference issues each op as its own kernel, kernels/bindings.cpp:90-99).
//
// Why: at batch 1 every op of a small model is latency-bound. A TinyLlama layer moves 23 MB of weights (2.9 us at
// 8 TB/s) but takes six launches of 3-6 us each, because each launch pays the launch gap and then a chain of
// dependent round trips (arguments, activation, weights) before its first FMA. Here the weights never sit on that
// chain: a workgroup requests the next phase's weight rows (and, for attention, its pages of K and V) while the
// current phase is still computing, and only the activation round trip and a grid barrier separate two phases.
//
// Grid: one workgroup of 8 waves per compute unit (all resident at once: the kernel is launched with at most as many
// workgroups as the device has CUs and a register and LDS budget of one workgroup per CU).
// Work split per phase (global wave gw of W = 8 x grid waves):
//   GEMV phases   wave gw owns rows [N gw / W, N (gw + 1) / W) (gate|up: pairs of interleaved rows) over the whole K;
//                 lane l takes the 32-weight columns l, l + 64, ... of each row, x comes from LDS (staged once per
//                 workgroup, transposed so that the lanes of a step read consecutive 16-byte words), the row is summed
//                 by DPP. The column arithmetic is the W4A16 GEMV's (w4_common.hpp): nibbles OR-ed into fp16 magic
//                 numbers, v_dot2_f32_f16, offsets and zero point removed once per column, exact products. Row
//                 results are gathered per workgroup in LDS and written with one coalesced store.
//   attention     workgroup u owns (kv head u % n_kv, split u / n_kv); split = 8 waves x nt 16-token tiles
//                 (part_size 128 nt); the lean MFMA arithmetic of paged_attention.hip (16 x 16 f16 tiles, p as fp16
//                 hi + lo, one online-softmax round per wave, waves merged in LDS), RoPE of q and k and the KV append
//                 by the split that owns *pos; one live split writes the output, else (o, m, l) partials.
//   combine       up to kFuseSplits partials: inside the o projection's operand staging (every workgroup merges them
//                 for its own copy); more: a phase of its own, wave h merging query head h.
// Every activation, residual and partial has its own slot per layer in the caller's work buffer, written once per
// launch (device-scope stores, write-through across the XCDs' L2s) before the barrier that precedes its reads, so no
// cache can hold an older copy and the reads are ordinary cached loads.
//
// Grid barrier, in two halves: arrival (every thread waits for its own stores, the workgroup meets at s_barrier,
// thread 0 adds 1 to its group's counter: workgroup % 32, 32 counters on separate 128-byte lines), then every wave
// issues the loads of a later phase, then the wait (wave 0 polls the counters until each has reached (barriers so
// far) x (workgroups of the group)). The poll is bounded: after kSpinLimit rounds (about a second) the waiting
// workgroup sets the abort word and every workgroup returns at its next poll, so a launch always ends. At the end
// every workgroup counts itself out; the last one writes *tok / *pos and zeroes every counter, so the next launch
// (e.g. the next graph replay) starts from zero.
#include "common.hpp"
#include "launch.hpp"
#include "w4_common.hpp"
#include "attn_common.hpp"
#include "dk_amd.h"

namespace dk {
namespace {

constexpr int kStepWaves = 8;
constexpr int kStepThreads = kStepWaves * kWave;
constexpr int kBarGroups = 32;     // arrival counters, one per group of workgroups (workgroup % 32)
constexpr int kSyncStride = 32;    // uint32 words between two sync words (one 128-byte line each)
constexpr int kSyncGroups = 8;     // argmax keys, one per group of workgroups (workgroup % 8)
constexpr int kSyncExit = kBarGroups * kSyncStride;
constexpr int kSyncAbort = kSyncExit + kSyncStride;
constexpr int kSyncKeys = kSyncAbort + kSyncStride;  // kSyncGroups uint64 argmax keys, kSyncStride words apart
static_assert(kSyncAbort == DK_STEP_SYNC_ABORT, "abort word of the public header");
static_assert(kSyncKeys + kSyncGroups * kSyncStride <= DK_STEP_SYNC_WORDS, "sync buffer size of the public header");
constexpr int kSpinLimit = 1 << 21;
constexpr int kWBudget = 4;  // 16-byte weight words per lane per batch of GEMV rows (more spills registers)

// ---- global-address-space views. Pointers read from the descriptor or the layer table are generic to the compiler;
// accesses through them would be flat instructions, which also count against lgkmcnt, so every LDS wait would wait
// for the weight loads in flight. Every access goes through these casts instead.
template <class T>
using gptr_t = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr_t<const T> gp(const T* p) {
  return (gptr_t<const T>)p;
}
template <class T>
__device__ __forceinline__ gptr_t<T> gpw(T* p) {
  return (gptr_t<T>)p;
}
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) { return __builtin_nontemporal_load(gp(p)); }

// ---- device-scope (agent) stores for data produced inside the launch (write-through: coherent across the XCDs)
__device__ __forceinline__ void st_coh32(void* p, uint32_t v) {
  __hip_atomic_store(gpw(reinterpret_cast<uint32_t*>(p)), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh64(void* p, uint64_t v) {
  __hip_atomic_store(gpw(reinterpret_cast<uint64_t*>(p)), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh128(void* p, u32x4 v) {
  st_coh64(p, (uint64_t)v[0] | ((uint64_t)v[1] << 32));
  st_coh64(reinterpret_cast<char*>(p) + 8, (uint64_t)v[2] | ((uint64_t)v[3] << 32));
}
__device__ __forceinline__ void st_coh16(f16* p, f16 v) {
  __hip_atomic_store(gpw(reinterpret_cast<uint16_t*>(p)), __builtin_bit_cast(uint16_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_cohf(float* p, float v) { st_coh32(p, __float_as_uint(v)); }

// ---- grid barrier (see the file header), in two halves so that loads issued between them (the next phase's weights)
// overlap the wait without delaying the arrival.
// Arrival: every thread's device-scope stores have completed (s_waitcnt 0: no load is outstanding at this point),
// then thread 0 adds 1 to its group's counter (32 counters on separate 128-byte lines, 8 workgroups each at 256).
__device__ __forceinline__ void grid_arrive(uint32_t* sync, uint32_t gen) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(&sync[(blockIdx.x % kBarGroups) * kSyncStride], 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Wait: lanes 0..31 of wave 0 poll the counters, lane 32 the abort word, until every counter has reached
// gen x (workgroups of its group). Returns false once the launch is aborted (a wait ran past kSpinLimit polls
// somewhere); the caller then returns.
__device__ bool grid_wait(uint32_t* sync, uint32_t gen, int* s_flag) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const int lane = tid, nblk = gridDim.x;
    uint32_t* p = lane < kBarGroups ? &sync[lane * kSyncStride] : &sync[kSyncAbort];
    const uint32_t need = lane < kBarGroups ? gen * (uint32_t)((nblk - lane + kBarGroups - 1) / kBarGroups) : 0u;
    int flag = 0;
    for (int it = 0;; ++it) {
      uint32_t v = 0;
      if (lane <= kBarGroups) v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t ab = __builtin_amdgcn_readlane(v, kBarGroups);
      const bool ok = lane < kBarGroups ? v >= need : true;
      if (ab != 0u) {
        flag = 1;
        break;
      }
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
      if (it >= kSpinLimit) {
        if (lane == 0) __hip_atomic_store(&sync[kSyncAbort], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) *s_flag = flag;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_flag) == 0;  // uniform: the caller returns or goes on as one
}

// ---- x staging: the K-vector operand of a GEMV phase, computed once per workgroup into LDS.
// Chunk j (8 fp16 values, 16 bytes) of x goes to xs[stage_index<TR>(j)]: for the INT4 GEMV (TR) column u = j / 4,
// word k = j % 4 sits at ((u / 64) * 4 + k) * 64 + u % 64, so that lane l of column step c reads word k of column
// 64 c + l at (4 c + k) * 64 + l (consecutive 16-byte words across the wave); for the fp16 head chunk j sits at j.
template <bool TR>
__device__ __forceinline__ int stage_index(int j) {
  if constexpr (TR) {
    const int u = j >> 2, k = j & 3;
    return (((u >> 6) << 2) + k) * kWave + (u & 63);
  } else {
    return j;
  }
}

template <int SCH>
struct StageRaw {
  u32x4 a[SCH];  // x
  u32x4 b[SCH];  // delta
  u32x4 c[SCH];  // norm weight
};

// Issues the operand loads: x, delta (both may have been produced in this launch: each such slot is written once per
// launch, before the barrier that precedes this read, so no cache holds an older copy), norm weight.
template <int SCH>
__device__ __forceinline__ void stage_issue(StageRaw<SCH>& r, const f16* x, const f16* delta, const f16* nw,
                                            int nchunks, int tid) {
#pragma unroll
  for (int i = 0; i < SCH; ++i) {
    const int j = tid + kStepThreads * i;
    if (j < nchunks) {
      r.a[i] = *gp(reinterpret_cast<const u32x4*>(x + 8 * j));
      if (delta != nullptr) r.b[i] = *gp(reinterpret_cast<const u32x4*>(delta + 8 * j));
      if (nw != nullptr) r.c[i] = *gp(reinterpret_cast<const u32x4*>(nw + 8 * j));
    }
  }
}

// The o projection's operand when the attention left nsplit (2 .. kFuseSplits) partials per head: chunk j (dims
// 8 (j % (D / 8)) .. + 8 of head j / (D / 8)) = sum_s w_s o_s / sum_s w_s l_s with w_s = e^(m_s - max_s m_s), the
// log-sum-exp combine of paged_attention.cu:366-427 (reference), computed by every workgroup for its own staging.
constexpr int kFuseSplits = 8;

template <int SCH, int D>
__device__ __forceinline__ void stage_combine(StageRaw<SCH>& r, const float* opart, const float* mpart,
                                              const float* lpart, int ms, int nsplit, int nchunks, int tid) {
#pragma unroll
  for (int i = 0; i < SCH; ++i) {
    const int j = tid + kStepThreads * i;
    if (j < nchunks) {
      const int head = j / (D / 8), d0 = (j % (D / 8)) * 8;
      float m[kFuseSplits], l[kFuseSplits];
      u32x4 oa[kFuseSplits], ob[kFuseSplits];
#pragma unroll
      for (int k = 0; k < kFuseSplits; ++k) {
        if (k < nsplit) {
          const size_t hs = (size_t)head * ms + k;
          m[k] = *gp(mpart + hs);
          l[k] = *gp(lpart + hs);
          oa[k] = *gp(reinterpret_cast<const u32x4*>(opart + hs * D + d0));
          ob[k] = *gp(reinterpret_cast<const u32x4*>(opart + hs * D + d0 + 4));
        }
      }
      float M = -INFINITY;
#pragma unroll
      for (int k = 0; k < kFuseSplits; ++k)
        if (k < nsplit) M = fmaxf(M, m[k]);
      float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kFuseSplits; ++k) {
        if (k < nsplit) {
          const float w = (m[k] == -INFINITY) ? 0.f : __expf(m[k] - M);
          L = fmaf(w, l[k], L);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[e] = fmaf(w, __uint_as_float(oa[k][e]), o[e]);
            o[4 + e] = fmaf(w, __uint_as_float(ob[k][e]), o[4 + e]);
          }
        }
      }
      const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) r.a[i][e] = as_u32(f16x2{(f16)(o[2 * e] * inv), (f16)(o[2 * e + 1] * inv)});
    }
  }
}

// Computes the operand into LDS. Without a norm weight: x as loaded. With one: the reference's add_rmsnorm
// (kernels/fused_norm.cu:8-54): xn = fp16(x + delta), r = 1 / sqrt(sum(float(xn)^2) / K + eps) over the whole vector,
// value = w * fp16(float(xn) * r) (fp16 product); x_out (workgroup 0 only) receives xn. Ends with a workgroup barrier.
template <int SCH, bool TR>
__device__ __forceinline__ void stage_finish(StageRaw<SCH>& r, bool has_delta, const f16* nw, float eps, int K,
                                             f16* x_out, u32x4* xs, float* red, int tid) {
  const int nchunks = K >> 3;
  if (nw == nullptr) {
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int j = tid + kStepThreads * i;
      if (j < nchunks) xs[stage_index<TR>(j)] = r.a[i];
    }
    __syncthreads();
    return;
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < SCH; ++i) {
    const int j = tid + kStepThreads * i;
    if (j < nchunks) {
      if (has_delta) {
#pragma unroll
        for (int e = 0; e < 4; ++e) r.a[i][e] = as_u32(as_f16x2(r.a[i][e]) + as_f16x2(r.b[i][e]));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(r.a[i][e]);
        const float a = (float)h.x, b = (float)h.y;
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
  ss = wave_sum_all(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kStepWaves; ++w) tot += red[w];
  const float rn = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
  for (int i = 0; i < SCH; ++i) {
    const int j = tid + kStepThreads * i;
    if (j < nchunks) {
      if (x_out != nullptr) st_coh128(x_out + 8 * j, r.a[i]);
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_f16x2(r.a[i][e]);
        const f16x2 hn = {(f16)((float)h.x * rn), (f16)((float)h.y * rn)};
        v[e] = as_u32(as_f16x2(r.c[i][e]) * hn);
      }
      xs[stage_index<TR>(j)] = v;
    }
  }
  __syncthreads();
}

// ---- INT4 GEMV rows of one wave
template <int C, int R>
struct W4Batch {
  u32x4 w[R][C];
  uint32_t s[R][C];
};

// Issues the weight and scale/zero loads of rows [row0, row0 + n) (n <= R, wave-uniform), C column steps each.
template <int C, int R>
__device__ __forceinline__ void w4_issue(W4Batch<C, R>& b, const void* W, const void* SZ, int row0, int n, int U,
                                         int gsh, int lane) {
  // wave-uniform row bases (scalar registers) plus 32-bit per-lane byte offsets: the global_load saddr + voffset form,
  // so no 64-bit per-lane address is ever kept live
  const int NG = U >> gsh;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < n) {
      const char* wb = reinterpret_cast<const char*>(W) + (size_t)(row0 + r) * U * sizeof(u32x4);
      const char* sb = reinterpret_cast<const char*>(SZ) + (size_t)(row0 + r) * NG * sizeof(uint32_t);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint32_t u = (uint32_t)min(64 * c + lane, U - 1);
        b.w[r][c] = ld_stream(reinterpret_cast<const u32x4*>(wb + u * (uint32_t)sizeof(u32x4)));
        b.s[r][c] = *gp(reinterpret_cast<const uint32_t*>(sb + (u >> gsh) * (uint32_t)sizeof(uint32_t)));
      }
    }
  }
}

// Row sums of a batch against the staged x (valid in lane 63).
template <int C, int R>
__device__ __forceinline__ void w4_rows(const W4Batch<C, R>& b, const u32x4* xs, int n, int U, int lane,
                                        float (&v)[R]) {
  const NibbleMasks m = nibble_masks();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if (64 * c < U) {
      u32x4 xc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) xc[k] = xs[(4 * c + k) * kWave + lane];
      const ColumnSums cs = column_sums(xc);
      const bool live = 64 * c + lane < U;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r < n) {
          const f16x2 sz = as_f16x2(b.s[r][c]);
          const float p = (float)sz.x * column_row(b.w[r][c], (float)sz.y, xc, cs, m);
          acc[r] += live ? p : 0.f;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = wave_sum_lane63(acc[r]);
}

// Output of a GEMV phase: plain rows (y[row] = fp16 sum) or SwiGLU pairs (rows 2i, 2i + 1 = gate_i, up_i;
// y[i] = silu_mul(fp16 gate, fp16 up), the rounding of kernels/fused_swiglu.cu:7-21).
enum { kEpiRows = 0, kEpiSwiglu = 1 };

// The wave's rows [row0, row0 + n): batch `a` was issued by the caller (rows row0 .. row0 + min(n, R)); later
// batches alternate between `a` and a second buffer (double buffering without register copies).
// Row results go to the workgroup's LDS gather buffer (index = output element - ob); w4_flush then writes the
// workgroup's contiguous output range with one coalesced device-scope store per thread, so each 128-byte line of an
// output vector receives a few wide writes instead of one 2-byte write per row.
template <int C, int R, int EPI>
__device__ __forceinline__ void w4_store(const float (&v)[R], int row, int nb, f16* s_out, int ob, int lane) {
  if (lane == 63) {
    if constexpr (EPI == kEpiRows) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (r < nb) s_out[row + r - ob] = (f16)v[r];
    } else {
#pragma unroll
      for (int r = 0; r + 1 < R; r += 2)
        if (r + 1 < nb) s_out[((row + r) >> 1) - ob] = silu_mul((f16)v[r], (f16)v[r + 1]);
    }
  }
}

template <int C, int R, int EPI>
__device__ __forceinline__ void w4_wave(W4Batch<C, R>& a, const void* W, const void* SZ, int row0, int n, int U,
                                        int gsh, const u32x4* xs, f16* s_out, int ob, int lane) {
  W4Batch<C, R> b;
  float v[R];
  for (int done = 0; done < n; done += 2 * R) {
    int nb = min(R, n - done), nn = min(R, n - done - R);
    if (nn > 0) w4_issue<C, R>(b, W, SZ, row0 + done + R, nn, U, gsh, lane);
    __builtin_amdgcn_sched_barrier(0);
    w4_rows<C, R>(a, xs, nb, U, lane, v);
    w4_store<C, R, EPI>(v, row0 + done, nb, s_out, ob, lane);
    if (nn <= 0) break;
    nb = nn;
    nn = min(R, n - done - 2 * R);
    if (nn > 0) w4_issue<C, R>(a, W, SZ, row0 + done + 2 * R, nn, U, gsh, lane);
    __builtin_amdgcn_sched_barrier(0);
    w4_rows<C, R>(b, xs, nb, U, lane, v);
    w4_store<C, R, EPI>(v, row0 + done + R, nb, s_out, ob, lane);
  }
}

// The workgroup's outputs [ob, ob + count) from the gather buffer to y.
__device__ __forceinline__ void w4_flush(const f16* s_out, f16* y, int ob, int count, int tid) {
  __syncthreads();
  if (tid < count) st_coh16(y + ob + tid, s_out[tid]);
}

// rows of wave gw of W when N rows (or N / 2 pairs) are split evenly
__device__ __forceinline__ void wave_rows(int N, bool pairs, int gw, int W, int& r0, int& n) {
  const long long units = pairs ? N / 2 : N;
  const int a = (int)(units * gw / W), b = (int)(units * (gw + 1) / W);
  r0 = pairs ? 2 * a : a;
  n = pairs ? 2 * (b - a) : b - a;
}

// ---- fp16 LM head rows of one wave: W fp16 [V, K], lane l holds chunks l, l + 64, ... (CF per row)
template <int CF, int R>
struct F16Batch {
  u32x4 w[R][CF];
};

template <int CF, int R>
__device__ __forceinline__ void f16_issue(F16Batch<CF, R>& b, const u32x4* __restrict__ W, int row0, int n, int UF,
                                          int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < n) {
      const char* wb = reinterpret_cast<const char*>(W) + (size_t)(row0 + r) * UF * sizeof(u32x4);
#pragma unroll
      for (int c = 0; c < CF; ++c)
        b.w[r][c] = ld_stream(reinterpret_cast<const u32x4*>(
            wb + (uint32_t)min(lane + 64 * c, UF - 1) * (uint32_t)sizeof(u32x4)));
    }
  }
}

// ---- attention (one workgroup per (kv head, split)); MfmaShape of paged_attention.hip's lean kernel
template <int D>
struct LeanShape {
  static constexpr int KW = D / 32;  // 16-byte K / q words per lane
  static constexpr int QS = D / 16;  // QK^T MFMA steps
  static constexpr int VD = D / 16;  // dims of a V row per lane (= P.V dim tiles)
  static constexpr int CPL = D / 8;  // 16-byte slices per head vector
};
constexpr int kAttnNT = 2;  // most 16-token tiles per wave (part_size 256)

template <int D>
struct AttnPre {  // issued before the barrier that precedes the attention phase
  int pg[kAttnNT];
  u32x4 kr[kAttnNT][LeanShape<D>::KW];
  VRow<LeanShape<D>::VD> vr[kAttnNT][4];
};

template <int D>
struct AttnQ {  // issued after that barrier: q, RoPE partners, the new k / v, the tables of *pos
  u32x4 qr[LeanShape<D>::KW], qp[LeanShape<D>::KW], ko[LeanShape<D>::KW], kp[LeanShape<D>::KW];
  VRow<LeanShape<D>::VD> vnew;
  float cs[LeanShape<D>::KW][8], sn[LeanShape<D>::KW][8];
};

template <int D>
struct AttnRot {  // rotated q slices, rotated new k, new v
  u32x4 qr[LeanShape<D>::KW], knew[LeanShape<D>::KW];
  VRow<LeanShape<D>::VD> vnew;
};

template <int VD>
__device__ __forceinline__ VRow<VD> ld_vrow(const f16* p) {
  VRow<VD> r;
  if constexpr (VD == 4) {
    const u32x2 v = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x2*>(p)));
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else {
    const u32x4 v = ld_stream(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = v[i];
  }
  return r;
}

// The layer table is copied into LDS at entry; a field is read back as a wave-uniform value (readfirstlane), so the
// weight addresses stay in scalar registers and no layer lookup waits on a vector load.
constexpr int kLayerFields = sizeof(dk_step_layer) / sizeof(void*);
enum {
  kLQkvW = 0, kLQkvS, kLOW, kLOS, kLGuW, kLGuS, kLDownW, kLDownS, kLLn1, kLLn2, kLKc, kLVc
};
static_assert(kLayerFields == 12, "dk_step_layer holds 12 pointers");
__device__ __forceinline__ const void* layer_ptr(const uint64_t* s_tab, int li, int field) {
  const uint64_t v = s_tab[li * kLayerFields + field];
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

struct StepDev {  // the descriptor as the kernel sees it
  dk_step_desc d;
  int log2P, gsh;
};

__device__ __forceinline__ size_t kv_row(int page, int t, int kvh, int n_kv, int log2P, int D) {
  return ((((size_t)page * n_kv + kvh) << log2P) + (t & ((1 << log2P) - 1))) * D;
}

template <int D>
__device__ __forceinline__ void attn_prefetch(AttnPre<D>& a, const StepDev& sd, const f16* kc, const f16* vc, int kvh,
                                              int split, int nt, bool live, int wave, int lane) {
  using S = LeanShape<D>;
  const dk_step_desc& d = sd.d;
  const int col = lane & 15, g = lane >> 4;
  const int t0 = split * d.part_size;
#pragma unroll
  for (int i = 0; i < kAttnNT; ++i) {
    const int tl = (wave + kStepWaves * i) << 4;
    const int lp = (t0 + tl) >> sd.log2P;
    const bool in = live && i < nt && lp < d.n_bt;
    const int e = *gp(d.bt + (in ? lp : 0));
    a.pg[i] = (in && e >= 0 && e < d.n_pages) ? e : -1;
  }
#pragma unroll
  for (int i = 0; i < kAttnNT; ++i) {
    const int ts = t0 + ((wave + kStepWaves * i) << 4);
    if (a.pg[i] >= 0) {
#pragma unroll
      for (int w = 0; w < S::KW; ++w)
        a.kr[i][w] = ld_stream(reinterpret_cast<const u32x4*>(
            kc + kv_row(a.pg[i], ts + col, kvh, d.n_kv, sd.log2P, D) + 8 * (4 * w + g)));
#pragma unroll
      for (int v = 0; v < 4; ++v)
        a.vr[i][v] = ld_vrow<S::VD>(vc + kv_row(a.pg[i], ts + 4 * g + v, kvh, d.n_kv, sd.log2P, D) + S::VD * col);
    } else {
#pragma unroll
      for (int w = 0; w < S::KW; ++w) a.kr[i][w] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int k = 0; k < S::VD / 2; ++k) a.vr[i][v].w[k] = 0u;
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void attn_issue_q(AttnQ<D>& q, const StepDev& sd, const f16* qkv, int kvh, int hpg, int pos,
                                             int lane) {
  using S = LeanShape<D>;
  const dk_step_desc& d = sd.d;
  const int col = lane & 15, g = lane >> 4;
  const bool qlive = col < hpg;
  const f16* qh = qkv + (size_t)(kvh * hpg + (qlive ? col : 0)) * D;
  const f16* kh = qkv + (size_t)(d.n_q + kvh) * D;
  const f16* vh = qkv + (size_t)(d.n_q + d.n_kv + kvh) * D;
#pragma unroll
  for (int w = 0; w < S::KW; ++w) {
    const int c = 4 * w + g, pc = (c + S::CPL / 2) % S::CPL;
    q.qr[w] = *gp(reinterpret_cast<const u32x4*>(qh + 8 * c));
    q.qp[w] = *gp(reinterpret_cast<const u32x4*>(qh + 8 * pc));
    q.ko[w] = *gp(reinterpret_cast<const u32x4*>(kh + 8 * c));
    q.kp[w] = *gp(reinterpret_cast<const u32x4*>(kh + 8 * pc));
  }
#pragma unroll
  for (int i = 0; i < S::VD / 2; ++i) q.vnew.w[i] = gp(reinterpret_cast<const uint32_t*>(vh + S::VD * col))[i];
#pragma unroll
  for (int w = 0; w < S::KW; ++w) {
    const int ti = (8 * (4 * w + g)) % (D / 2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q.cs[w][e] = gp(d.cos_t)[(size_t)pos * (D / 2) + ti + e];
      q.sn[w][e] = gp(d.sin_t)[(size_t)pos * (D / 2) + ti + e];
    }
  }
}

// RoPE of q (the workgroup's heads, zero for the unused MFMA columns) and of the new k (rotate_half, fp32 tables,
// reference/ref_ops.py:36-53 rounding).
template <int D>
__device__ __forceinline__ AttnRot<D> attn_rope(const AttnQ<D>& q, int hpg, int lane) {
  using S = LeanShape<D>;
  const int col = lane & 15, g = lane >> 4;
  AttnRot<D> r;
#pragma unroll
  for (int w = 0; w < S::KW; ++w) {
    const int c = 4 * w + g;
    r.qr[w] = col < hpg ? rope_slice<D>(q.qr[w], q.qp[w], q.cs[w], q.sn[w], c < S::CPL / 2) : u32x4{0u, 0u, 0u, 0u};
    r.knew[w] = rope_slice<D>(q.ko[w], q.kp[w], q.cs[w], q.sn[w], c < S::CPL / 2);
  }
  r.vnew = q.vnew;
  return r;
}

// The split of workgroup (kvh, split): RoPE, append (owner split), scores, softmax, P.V, merge of the 8 waves, output
// or partials. LDS: s_m, s_l, s_w [8][8] and s_o [8][8][D] floats at lds.
template <int D>
__device__ __forceinline__ void attn_finish(AttnPre<D>& a, const AttnRot<D>& q, const StepDev& sd, f16* kc, f16* vc,
                                            int kvh, int split, int nt, int hpg, int pos, int ctx, int nsplit,
                                            f16* out, float* o_part, float* m_part, float* l_part, float* lds,
                                            int wave, int lane, int tid) {
  using S = LeanShape<D>;
  constexpr int KW = S::KW, QS = S::QS, VD = S::VD;
  const dk_step_desc& d = sd.d;
  float (*s_m)[8] = reinterpret_cast<float (*)[8]>(lds);
  float (*s_l)[8] = reinterpret_cast<float (*)[8]>(lds + 64);
  float (*s_w)[8] = reinterpret_cast<float (*)[8]>(lds + 128);
  float (*s_o)[8][D] = reinterpret_cast<float (*)[8][D]>(lds + 192);
  const int col = lane & 15, g = lane >> 4;
  const int PS = d.part_size;
  const int t0 = split * PS;
  const u32x4(&qr)[KW] = q.qr;
  const u32x4(&knew)[KW] = q.knew;
  // append: the split that owns token pos (the last live split when the cap is below pos)
  const int owner = min(pos / PS, nsplit - 1);
  if (split == owner && wave == 0) {
    const int lp = pos >> sd.log2P;
    const int page = lp < d.n_bt ? *gp(d.bt + lp) : -1;
    if (page >= 0 && page < d.n_pages) {
      const size_t row = kv_row(page, pos, kvh, d.n_kv, sd.log2P, D);
      if (col == 0) {
#pragma unroll
        for (int w = 0; w < KW; ++w) *gpw(reinterpret_cast<u32x4*>(kc + row + 8 * (4 * w + g))) = knew[w];
      }
      if (g == 0) {
#pragma unroll
        for (int i = 0; i < VD / 2; ++i) gpw(reinterpret_cast<uint32_t*>(vc + row + VD * col))[i] = q.vnew.w[i];
      }
    }
  }
  const int t1 = min(ctx, t0 + PS);
  const bool pos_here = pos >= t0 && pos < t1;
  const float scale = 1.0f / sqrtf((float)D);
  f4 sc[kAttnNT];
  float rmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < kAttnNT; ++i) {
    sc[i] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (i < nt) {
      const int ts = t0 + ((wave + kStepWaves * i) << 4);
      const bool tile = a.pg[i] >= 0;
      if (pos_here && tile && ts + col == pos) {
#pragma unroll
        for (int w = 0; w < KW; ++w) a.kr[i][w] = knew[w];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (pos_here && tile && ts + 4 * g + v == pos) a.vr[i][v] = q.vnew;
#pragma unroll
      for (int v = 0; v < 4; ++v) {  // rows past the context: zero V (a stale row must not reach p . V as NaN)
        const bool keep = tile && ts + 4 * g + v < t1;
#pragma unroll
        for (int k = 0; k < VD / 2; ++k) a.vr[i][v].w[k] = keep ? a.vr[i][v].w[k] : 0u;
      }
      f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        const int i0 = 2 * s, i1 = 2 * s + 1;
        c = mfma16(as_h4(a.kr[i][i0 >> 2][i0 & 3], a.kr[i][i1 >> 2][i1 & 3]),
                   as_h4(qr[i0 >> 2][i0 & 3], qr[i1 >> 2][i1 & 3]), c);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const bool live = tile && ts + 4 * g + v < t1;
        sc[i][v] = live ? c[v] * scale : -INFINITY;
        rmax = fmaxf(rmax, sc[i][v]);
      }
    }
  }
  const float m = rows_max(rmax);
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < kAttnNT; ++i) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float pv = (sc[i][v] == -INFINITY) ? 0.f : __expf(sc[i][v] - m);
      sc[i][v] = pv;
      ps += pv;
    }
  }
  const float l = rows_sum(ps);
  f4 acc[VD];
#pragma unroll
  for (int t = 0; t < VD; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kAttnNT; ++i) {
    if (i < nt) {
      h4 phi, plo;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        phi[v] = (f16)sc[i][v];
        plo[v] = (f16)(sc[i][v] - (float)phi[v]);
      }
#pragma unroll
      for (int t = 0; t < VD; ++t) {
        const int wi = t >> 1;
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(a.vr[i][1].w[wi], a.vr[i][0].w[wi], sel);
        const uint32_t hi = __builtin_amdgcn_perm(a.vr[i][3].w[wi], a.vr[i][2].w[wi], sel);
        const h4 vb = as_h4(lo, hi);
        acc[t] = mfma16(phi, vb, acc[t]);
        acc[t] = mfma16(plo, vb, acc[t]);
      }
    }
  }
  if (g == 0 && col < hpg) {
    s_m[wave][col] = m;
    s_l[wave][col] = l;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int hh = 4 * g + v;
    if (hh < hpg) {
#pragma unroll
      for (int t = 0; t < VD; ++t) s_o[wave][hh][VD * col + t] = acc[t][v];
    }
  }
  __syncthreads();
  float Mh = -INFINITY, Lh = 0.f;
  if (tid < hpg) {
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) Mh = fmaxf(Mh, s_m[w][tid]);
    float ww[kStepWaves];
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) {
      ww[w] = (s_m[w][tid] == -INFINITY) ? 0.f : __expf(s_m[w][tid] - Mh);
      Lh = fmaf(ww[w], s_l[w][tid], Lh);
    }
    const float inv = nsplit == 1 ? (Lh > 0.f ? 1.0f / Lh : 0.f) : 1.0f;
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) s_w[w][tid] = ww[w] * inv;
  }
  __syncthreads();
  for (int o = tid; o < hpg * D; o += kStepThreads) {
    const int hh = o / D, dd = o % D;
    float O = 0.f;
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) O = fmaf(s_w[w][hh], s_o[w][hh][dd], O);
    const int head = kvh * hpg + hh;
    if (nsplit == 1)
      st_coh16(out + (size_t)head * D + dd, (f16)O);
    else
      st_cohf(o_part + ((size_t)head * d.max_splits + split) * D + dd, O);
  }
  if (nsplit > 1 && tid < hpg) {
    const int head = kvh * hpg + tid;
    st_cohf(m_part + (size_t)head * d.max_splits + split, Mh);
    st_cohf(l_part + (size_t)head * d.max_splits + split, Lh);
  }
}

// Combine of query head `head` (one wave; lane owns dims D / 64 * lane ..): M = max m_s, w_s = e^(m_s - M),
// out = sum_s w_s o_s / sum_s w_s l_s (paged_attention.cu:366-427 of the reference).
template <int D>
__device__ __forceinline__ void combine_head(const float* o_part, const float* m_part, const float* l_part,
                                             int max_splits, f16* attn, int head, int nsplit, int lane) {
  constexpr int DPL = D / kWave;
  const float* mp = m_part + (size_t)head * max_splits;
  const float* lp = l_part + (size_t)head * max_splits;
  const float* op = o_part + (size_t)head * max_splits * D + DPL * lane;
  const bool sl = lane < nsplit;
  const float ms = sl ? *gp(mp + lane) : -INFINITY;
  const float ls = sl ? *gp(lp + lane) : 0.f;
  float M = ms;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, kWave));
  const float ws = (ms == -INFINITY) ? 0.f : __expf(ms - M);
  float L = ws * ls;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, kWave);
  float acc[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) acc[k] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    float ov[8][DPL];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int k = 0; k < DPL; ++k) ov[s][k] = s0 + s < nsplit ? *gp(op + (size_t)(s0 + s) * D + k) : 0.f;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float w =
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), min(s0 + s, 63)));
#pragma unroll
      for (int k = 0; k < DPL; ++k) acc[k] = s0 + s < nsplit ? fmaf(w, ov[s][k], acc[k]) : acc[k];
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  f16* out = attn + (size_t)head * D + DPL * lane;
  if constexpr (DPL == 1) {
    st_coh16(out, (f16)(acc[0] * inv));
  } else {
    st_coh32(out, as_u32(f16x2{(f16)(acc[0] * inv), (f16)(acc[1] * inv)}));
  }
}

// ---- the kernel. D: head dim; CH / CI: most 64-column steps of a row for K = H / K = I; CF: most 64-chunk steps of
// an fp16 head row (K = H).
template <int D, int CH, int CI, int CF>
struct StepCfg {
  static constexpr int RH = kWBudget / CH >= 2 ? kWBudget / CH : 2;  // rows per batch, K = H (INT4 head)
  static constexpr int RQ = CH == 1 ? 2 : 4;                         // qkv rows per batch
  static constexpr int RO = 2;                                       // o rows per batch
  static constexpr int RG = CH == 1 ? 6 : 4;                         // gate|up rows per batch (even: pairs)
  static constexpr int RI = kWBudget / CI >= 1 ? kWBudget / CI : 1;  // rows per batch, K = I
  static constexpr int RF = kWBudget / CF >= 1 ? kWBudget / CF : 1;  // rows per batch, fp16 head
  static constexpr int SH = (CH + 1) / 2;                            // staging chunks per thread, K = H
  static constexpr int SI = (CI + 1) / 2;                            // K = I
  static constexpr int SF = (CF + 7) / 8;                            // fp16 head
};

template <int D, int CH, int CI, int CF>
__global__ void __launch_bounds__(kStepThreads, 1) decode_step_kernel(const StepDev sd) {
  using Cfg = StepCfg<D, CH, CI, CF>;
  constexpr int RH = Cfg::RH, RI = Cfg::RI, RF = Cfg::RF, RQ = Cfg::RQ, RO = Cfg::RO, RG = Cfg::RG;
  extern __shared__ u32x4 lds[];
  __shared__ float s_red[kStepWaves];
  __shared__ unsigned long long s_key[kStepWaves];
  __shared__ int s_flag;
  __shared__ f16 s_out[kStepOutMax];
  __shared__ uint64_t s_tab[kStepMaxLayers * kLayerFields];
  const dk_step_desc& d = sd.d;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = gridDim.x * kStepWaves, gw = blockIdx.x * kStepWaves + wave;
  const int H = d.hidden, I = d.inter, n_q = d.n_q, n_kv = d.n_kv, hpg = n_q / n_kv;
  const int gsh = sd.gsh;
  const int UH = H >> 5, UI = I >> 5;
  uint32_t* sync = d.sync;

  const int pos = *d.pos;
  if (pos < 0 || pos >= d.max_pos) return;  // uniform over the grid: nothing is touched
  const long long cap = (long long)d.n_bt << sd.log2P;
  const int ctx = (int)((long long)pos + 1 < cap ? (long long)pos + 1 : cap);
  const int nsplit = attn_splits(ctx, d.part_size, d.max_splits);
  const int nt = d.part_size >> 7;
  const long long tok0 = *d.tok;
  const bool tok_ok = tok0 >= 0 && tok0 < d.vocab;
  const StepLayout LY = step_layout(H, n_q, n_kv, D, I, d.max_splits);
  for (int i = tid; i < d.n_layers * kLayerFields; i += kStepThreads)
    s_tab[i] = gp(reinterpret_cast<const uint64_t*>(d.layers))[i];
  __syncthreads();

  // this workgroup's attention unit and this wave's rows in each GEMV phase
  const int akvh = blockIdx.x % n_kv, asplit = blockIdx.x / n_kv;
  const bool alive = asplit < nsplit;
  const int NQKV = (n_q + 2 * n_kv) * D;
  int q0, qn, o0, on, g0, gn, d0, dn, h0, hn;
  wave_rows(NQKV, false, gw, W, q0, qn);
  wave_rows(H, false, gw, W, o0, on);
  wave_rows(2 * I, true, gw, W, g0, gn);
  wave_rows(H, false, gw, W, d0, dn);
  wave_rows(d.vocab, false, gw, W, h0, hn);
  // the workgroup's output ranges (its waves' ranges are consecutive): start and count of qkv, H-row and act outputs
  const int b0 = blockIdx.x * kStepWaves, b1 = b0 + kStepWaves;
  const int bq = (int)((long long)NQKV * b0 / W), bqn = (int)((long long)NQKV * b1 / W) - bq;
  const int bh = (int)((long long)H * b0 / W), bhn = (int)((long long)H * b1 / W) - bh;
  const int bi = (int)((long long)I * b0 / W), bin = (int)((long long)I * b1 / W) - bi;
  const bool head_int4 = d.head_sz != nullptr;

  uint32_t gen = 0;
  char* const work = reinterpret_cast<char*>(d.work);

  // loads issued ahead: the qkv rows and the attention pages of layer 0
  W4Batch<CH, RQ> pq;
  AttnPre<D> ap;
  w4_issue<CH, RQ>(pq, layer_ptr(s_tab, 0, kLQkvW), layer_ptr(s_tab, 0, kLQkvS), q0, min(qn, RQ), UH, gsh, lane);
  attn_prefetch<D>(ap, sd, reinterpret_cast<const f16*>(layer_ptr(s_tab, 0, kLKc)),
                   reinterpret_cast<const f16*>(layer_ptr(s_tab, 0, kLVc)), akvh, asplit, nt, alive, wave, lane);

  // Per layer: qkv | attention | [combine] | o | gate|up | down, a grid barrier after each phase. Between the arrival
  // and the wait of a barrier every wave issues the loads of a later phase: the o and gate|up rows after the attention,
  // the down rows after o, the next layer's qkv rows after gate|up, its attention pages after down.
  for (int li = 0; li < d.n_layers; ++li) {
    // the lane indices are redefined (as far as the compiler knows) every layer, so per-lane address arithmetic is
    // recomputed where it is used instead of being hoisted out of the loop into spilled registers
    int ln = lane, tl = tid;
    asm volatile("" : "+v"(ln), "+v"(tl));
    f16* kc = const_cast<f16*>(reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLKc)));
    f16* vc = const_cast<f16*>(reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLVc)));
    char* const wl = work + (size_t)li * LY.layer;
    f16* const xq = reinterpret_cast<f16*>(wl + LY.xq);
    f16* const xg = reinterpret_cast<f16*>(wl + LY.xg);
    f16* const qkv = reinterpret_cast<f16*>(wl + LY.qkv);
    f16* const attn = reinterpret_cast<f16*>(wl + LY.attn);
    f16* const ob = reinterpret_cast<f16*>(wl + LY.o);
    f16* const act = reinterpret_cast<f16*>(wl + LY.act);
    f16* const down = reinterpret_cast<f16*>(wl + LY.down);
    float* const opart = reinterpret_cast<float*>(wl + LY.opart);
    float* const mpart = reinterpret_cast<float*>(wl + LY.mpart);
    float* const lpart = reinterpret_cast<float*>(wl + LY.lpart);
    // ---------------- qkv = W_qkv . rmsnorm(x + delta)   (layer 0: x = emb[tok], no delta); xq <- x + delta
    {
      StageRaw<Cfg::SH> st;
      const f16* xin;
      const f16* dl;
      if (li == 0) {
        xin = reinterpret_cast<const f16*>(d.emb) + (size_t)(tok_ok ? tok0 : 0) * H;
        dl = nullptr;
      } else {
        const char* wp = work + (size_t)(li - 1) * LY.layer;
        xin = reinterpret_cast<const f16*>(wp + LY.xg);
        dl = reinterpret_cast<const f16*>(wp + LY.down);
      }
      stage_issue<Cfg::SH>(st, xin, dl, reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLLn1)), H >> 3, tl);
      if (li == 0 && !tok_ok) {
#pragma unroll
        for (int i = 0; i < Cfg::SH; ++i) st.a[i] = u32x4{0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};
      }
      stage_finish<Cfg::SH, true>(st, dl != nullptr, reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLLn1)), d.eps,
                                  H,
                                  blockIdx.x == 0 ? xq : nullptr, lds, s_red, tl);
      w4_wave<CH, RQ, kEpiRows>(pq, layer_ptr(s_tab, li, kLQkvW),
                                layer_ptr(s_tab, li, kLQkvS), q0, qn, UH, gsh, lds, s_out, bq, ln);
      w4_flush(s_out, qkv, bq, bqn, tl);
    }
    grid_arrive(sync, ++gen);
    if (!grid_wait(sync, gen, &s_flag)) return;
    // ---------------- attention (RoPE, append, split) -> attn (one split) or the partials
    if (alive) {
      AttnQ<D> aq;
      attn_issue_q<D>(aq, sd, qkv, akvh, hpg, pos, ln);
      const AttnRot<D> rot = attn_rope<D>(aq, hpg, ln);
      attn_finish<D>(ap, rot, sd, kc, vc, akvh, asplit, nt, hpg, pos, ctx, nsplit, attn, opart, mpart, lpart,
                     reinterpret_cast<float*>(lds), wave, ln, tl);
    }
    grid_arrive(sync, ++gen);
    W4Batch<CH, RO> po;
    W4Batch<CH, RG> pg;
    w4_issue<CH, RO>(po, layer_ptr(s_tab, li, kLOW), layer_ptr(s_tab, li, kLOS), o0,
                     min(on, RO), UH, gsh, ln);
    w4_issue<CH, RG>(pg, layer_ptr(s_tab, li, kLGuW), layer_ptr(s_tab, li, kLGuS), g0,
                     min(gn, RG), UH, gsh, ln);
    if (!grid_wait(sync, gen, &s_flag)) return;
    // ---------------- combine of many partials as a phase of its own (few partials: inside the o staging)
    if (nsplit > kFuseSplits) {
      if (gw < n_q) combine_head<D>(opart, mpart, lpart, d.max_splits, attn, gw, nsplit, ln);
      grid_arrive(sync, ++gen);
      if (!grid_wait(sync, gen, &s_flag)) return;
    }
    // ---------------- o = W_o . attn
    {
      StageRaw<Cfg::SH> so;
      if (nsplit > 1 && nsplit <= kFuseSplits)
        stage_combine<Cfg::SH, D>(so, opart, mpart, lpart, d.max_splits, nsplit, H >> 3, tl);
      else
        stage_issue<Cfg::SH>(so, attn, nullptr, nullptr, H >> 3, tl);
      stage_finish<Cfg::SH, true>(so, false, nullptr, d.eps, H, nullptr, lds, s_red, tl);
      w4_wave<CH, RO, kEpiRows>(po, layer_ptr(s_tab, li, kLOW),
                                layer_ptr(s_tab, li, kLOS), o0, on, UH, gsh, lds, s_out, bh, ln);
      w4_flush(s_out, ob, bh, bhn, tl);
    }
    grid_arrive(sync, ++gen);
    W4Batch<CI, RI> pdn;
    w4_issue<CI, RI>(pdn, layer_ptr(s_tab, li, kLDownW), layer_ptr(s_tab, li, kLDownS),
                     d0, min(dn, RI), UI, gsh, ln);
    if (!grid_wait(sync, gen, &s_flag)) return;
    // ---------------- act = swiglu(W_gu . rmsnorm(xq + o)); xg <- xq + o
    {
      StageRaw<Cfg::SH> sg;
      stage_issue<Cfg::SH>(sg, xq, ob, reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLLn2)), H >> 3, tl);
      stage_finish<Cfg::SH, true>(sg, true, reinterpret_cast<const f16*>(layer_ptr(s_tab, li, kLLn2)), d.eps, H,
                                  blockIdx.x == 0 ? xg : nullptr, lds, s_red, tl);
      w4_wave<CH, RG, kEpiSwiglu>(pg, layer_ptr(s_tab, li, kLGuW),
                                  layer_ptr(s_tab, li, kLGuS), g0, gn, UH, gsh, lds, s_out, bi, ln);
      w4_flush(s_out, act, bi, bin, tl);
    }
    grid_arrive(sync, ++gen);
    if (li + 1 < d.n_layers) {
      w4_issue<CH, RQ>(pq, layer_ptr(s_tab, li + 1, kLQkvW), layer_ptr(s_tab, li + 1, kLQkvS),
                       q0, min(qn, RQ), UH, gsh, ln);
    }
    if (!grid_wait(sync, gen, &s_flag)) return;
    // ---------------- down = W_down . act
    {
      StageRaw<Cfg::SI> sa;
      stage_issue<Cfg::SI>(sa, act, nullptr, nullptr, I >> 3, tl);
      stage_finish<Cfg::SI, true>(sa, false, nullptr, d.eps, I, nullptr, lds, s_red, tl);
      w4_wave<CI, RI, kEpiRows>(pdn, layer_ptr(s_tab, li, kLDownW),
                                layer_ptr(s_tab, li, kLDownS), d0, dn, UI, gsh, lds, s_out, bh, ln);
      w4_flush(s_out, down, bh, bhn, tl);
    }
    grid_arrive(sync, ++gen);
    if (li + 1 < d.n_layers) {
      attn_prefetch<D>(ap, sd, reinterpret_cast<const f16*>(layer_ptr(s_tab, li + 1, kLKc)),
                       reinterpret_cast<const f16*>(layer_ptr(s_tab, li + 1, kLVc)), akvh, asplit,
                       nt, alive, wave, ln);
    }
    if (!grid_wait(sync, gen, &s_flag)) return;
  }

  const char* wlast = work + (size_t)(d.n_layers - 1) * LY.layer;
  const f16* xfin = reinterpret_cast<const f16*>(wlast + LY.xg);
  const f16* dfin = reinterpret_cast<const f16*>(wlast + LY.down);
  // ---------------- logits = head . rmsnorm(x + down); argmax
  unsigned long long best = 0;
  f16* logits = reinterpret_cast<f16*>(d.logits);
  if (!head_int4) {
    const int UF = H >> 3;
    const u32x4* Wf = reinterpret_cast<const u32x4*>(d.head_w);
    F16Batch<CF, RF> cb;
    StageRaw<Cfg::SF> sh;
    stage_issue<Cfg::SF>(sh, xfin, dfin,
                         reinterpret_cast<const f16*>(d.norm_f), UF, tid);
    f16_issue<CF, RF>(cb, Wf, h0, min(hn, RF), UF, lane);
    stage_finish<Cfg::SF, false>(sh, true, reinterpret_cast<const f16*>(d.norm_f), d.eps, H, nullptr, lds, s_red, tid);
    u32x4 xc[CF];
#pragma unroll
    for (int c = 0; c < CF; ++c) xc[c] = lds[min(lane + 64 * c, UF - 1)];
    for (int done = 0; done < hn; done += RF) {
      const int nb = min(RF, hn - done), nn = min(RF, hn - done - RF);
      F16Batch<CF, RF> nx;
      if (nn > 0) f16_issue<CF, RF>(nx, Wf, h0 + done + RF, nn, UF, lane);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < RF; ++r) {
        if (r < nb) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < CF; ++c) {
            float p = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) p = dot2(as_f16x2(cb.w[r][c][e]), as_f16x2(xc[c][e]), p);
            acc += lane + 64 * c < UF ? p : 0.f;
          }
          acc = wave_sum_lane63(acc);
          if (lane == 63) {
            const f16 y = (f16)acc;
            logits[h0 + done + r] = y;
            best = max(best, (unsigned long long)argmax_key((float)y, h0 + done + r));
          }
        }
      }
      if (nn > 0) cb = nx;
    }
  } else {
    const u32x4* Wq = reinterpret_cast<const u32x4*>(d.head_w);
    const uint32_t* Sq = reinterpret_cast<const uint32_t*>(d.head_sz);
    W4Batch<CH, RH> cb;
    StageRaw<Cfg::SH> sh;
    stage_issue<Cfg::SH>(sh, xfin, dfin,
                         reinterpret_cast<const f16*>(d.norm_f), H >> 3, tid);
    w4_issue<CH, RH>(cb, Wq, Sq, h0, min(hn, RH), UH, gsh, lane);
    stage_finish<Cfg::SH, true>(sh, true, reinterpret_cast<const f16*>(d.norm_f), d.eps, H, nullptr, lds, s_red, tid);
    for (int done = 0; done < hn; done += RH) {
      const int nb = min(RH, hn - done), nn = min(RH, hn - done - RH);
      W4Batch<CH, RH> nx;
      if (nn > 0) w4_issue<CH, RH>(nx, Wq, Sq, h0 + done + RH, nn, UH, gsh, lane);
      __builtin_amdgcn_sched_barrier(0);
      float v[RH];
      w4_rows<CH, RH>(cb, lds, nb, UH, lane, v);
      if (lane == 63) {
#pragma unroll
        for (int r = 0; r < RH; ++r) {
          if (r < nb) {
            const f16 y = (f16)v[r];
            logits[h0 + done + r] = y;
            best = max(best, (unsigned long long)argmax_key((float)y, h0 + done + r));
          }
        }
      }
      if (nn > 0) cb = nx;
    }
  }
  // workgroup's best key -> the group's key (device-scope max); then count out; the last workgroup finishes the step
  {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)best, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(best >> 32), 63);
    best = ((unsigned long long)hi << 32) | lo;
  }
  if (lane == 0) s_key[wave] = best;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kStepWaves; ++w) best = max(best, s_key[w]);
    unsigned long long* key = reinterpret_cast<unsigned long long*>(&sync[kSyncKeys + (blockIdx.x % kSyncGroups) *
                                                                           kSyncStride]);
    const unsigned long long seen = __hip_atomic_fetch_max(key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(seen));
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev = __hip_atomic_fetch_add(&sync[kSyncExit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) {
      unsigned long long k = 0;
      for (int g = 0; g < kSyncGroups; ++g) {
        unsigned long long* kg = reinterpret_cast<unsigned long long*>(&sync[kSyncKeys + g * kSyncStride]);
        k = max(k, (unsigned long long)__hip_atomic_load(kg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        __hip_atomic_store(kg, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *d.tok = (int64_t)(uint32_t)~(uint32_t)k;
      *d.pos = pos + 1;
      for (int g = 0; g < kBarGroups; ++g)
        __hip_atomic_store(&sync[g * kSyncStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sync[kSyncExit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int D, int CH, int CI, int CF>
size_t step_lds_bytes(int H, int I) {
  const size_t xs = (size_t)((max(H, I) / 32 + 63) / 64) * 4 * 64 * 16;
  const size_t xf = (size_t)((H / 8 + 63) / 64) * 64 * 16;
  const size_t at = (size_t)(192 + 8 * 8 * D) * sizeof(float);
  return max(max(xs, xf), at);
}

template <int D, int CH, int CI, int CF>
int launch_step_t(const StepDev& sd, int grid, hipStream_t st) {
  const size_t lds = step_lds_bytes<D, CH, CI, CF>(sd.d.hidden, sd.d.inter);
  hipLaunchKernelGGL((decode_step_kernel<D, CH, CI, CF>), dim3(grid), dim3(kStepThreads), lds, st, sd);
  return 0;
}

}  // namespace

// Limits of the two instances (head_dim 64: H <= 2048, I <= 6144; head_dim 128: H <= 4096, I <= 14336).
bool decode_step_fits(int head_dim, int H, int I) {
  if (head_dim == 64) return H <= 2048 && I <= 6144;
  if (head_dim == 128) return H <= 4096 && I <= 14336;
  return false;
}

// One workgroup per CU, provided the occupancy calculator confirms that a CU holds one (so every workgroup of the
// launch is resident at once and the grid barriers can complete). Cached per device.
int decode_step_grid(int head_dim) {
  static int cache[2][64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  const int t = head_dim == 128 ? 1 : 0;
  if (cache[t][dev] != 0) return cache[t][dev];
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return -1;
  const hipError_t e =
      t ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<128, 2, 7, 8>, kStepThreads,
                                                       step_lds_bytes<128, 2, 7, 8>(4096, 14336))
        : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<64, 1, 3, 4>, kStepThreads,
                                                       step_lds_bytes<64, 1, 3, 4>(2048, 6144));
  if (e != hipSuccess || per_cu < 1) return -1;
  cache[t][dev] = cus;
  return cus;
}

int launch_decode_step(const dk_step_desc& d, int grid, hipStream_t st) {
  StepDev sd;
  sd.d = d;
  int l = 0;
  while ((1 << l) < d.page) ++l;
  sd.log2P = l;
  int gl = 0;
  while ((1 << gl) < d.group) ++gl;
  sd.gsh = gl - 5;
  if (d.head_dim == 64) return launch_step_t<64, 1, 3, 4>(sd, grid, st);
  return launch_step_t<128, 2, 7, 8>(sd, grid, st);
}

}  // namespace dk
