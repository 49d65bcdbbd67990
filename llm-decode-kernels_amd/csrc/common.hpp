// Shared device helpers for the gfx950 (CDNA4, wave64) decode kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dk {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ f16x2 as_f16x2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// 16-byte load that bypasses cache retention: weights and KV rows are read once per token.
__device__ __forceinline__ u32x4 load_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }

// Write-through stores (agent-scope relaxed: `sc1`): the issuing XCD's L2 passes the data on to memory at once
// instead of holding the lines dirty until the write-back at the end of the kernel. They order nothing. Used for
// outputs of whole 128-byte lines that the next launch reads from every XCD (the attention split partials, the
// residual written by a norm prologue): 1.3-3 us per TinyLlama token in the decode step. Not for the GEMVs' 2-byte
// outputs, whose lines are written piecewise by several workgroups: write-through there cost 8.6 us per token.
__device__ __forceinline__ void store_through(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at byte offset `off` of `base` (a raw buffer store with the sc1 cache policy, bit 4 of its aux operand)
__device__ __forceinline__ void store_through16(void* base, uint32_t off, u32x4 v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 16);
}

// A constant moved into a VGPR behind an empty asm, so the optimiser treats it as a per-lane value. Used for the
// nibble masks of the INT4 dequant: with the mask and the OR constant both literal the compiler emits v_and_b32 +
// v_or_b32 (a gfx9 VOP3 instruction takes no literal and at most one scalar operand); with the mask in a VGPR it
// emits one v_and_or_b32. Build it once, ahead of the loops that use it.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Sum / max over aligned groups of WIDTH consecutive lanes (WIDTH a power of two <= 64); every lane of the group
// ends with the group result.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Reduction over the lanes that share (lane % STRIDE), i.e. xor offsets STRIDE, 2*STRIDE, ..., 32.
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float v) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int STRIDE>
__device__ __forceinline__ float strided_max(float v) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Full-wave sum through DPP (no LDS traffic, a few cycles per step): quad_perm [1,0,3,2] and [2,3,0,1] sum the quad,
// row_half_mirror and row_mirror the 16-lane row, row_bcast15 into rows 1 and 3 and row_bcast31 into rows 2 and 3
// carry the row sums upward. The total is valid in lane 63 only. Must be called with every lane of the wave active
// (the DPP source of an inactive lane is not defined); select 0 for dead lanes before calling.
#define DK_DPP_F32(v, ctrl, row_mask) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), (row_mask), 0xF, false))
__device__ __forceinline__ float wave_sum_lane63(float v) {
  v += DK_DPP_F32(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]
  v += DK_DPP_F32(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]
  v += DK_DPP_F32(v, 0x141, 0xF);  // row_half_mirror
  v += DK_DPP_F32(v, 0x140, 0xF);  // row_mirror
  v += DK_DPP_F32(v, 0x142, 0xA);  // row_bcast15, rows 1 and 3
  v += DK_DPP_F32(v, 0x143, 0xC);  // row_bcast31, rows 2 and 3
  return v;
}
// Sum over aligned groups of CPL = 8 or 16 consecutive lanes, every lane of the group ends with the group sum
// (quad_perm x2, row_half_mirror, and row_mirror for 16).
template <int CPL>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(CPL == 8 || CPL == 16, "group of 8 or 16 lanes");
  v += DK_DPP_F32(v, 0xB1, 0xF);
  v += DK_DPP_F32(v, 0x4E, 0xF);
  v += DK_DPP_F32(v, 0x141, 0xF);
  if constexpr (CPL == 16) v += DK_DPP_F32(v, 0x140, 0xF);
  return v;
}
// Transposed reduction of n = 2^k row partials per lane over each 16-lane DPP row ("row fold"). Summing every row
// over the wave separately costs 6 DPP steps per row; folding them together costs n - 1 DPP adds in all. Step s
// (s = 1..4) pairs lane L with lane L ^ X_s, X = {1, 2, 7, 15} (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), and merges two half-blocks of rows that differ in row bit s - 1: the lane keeps the
// half whose bit equals its c_s and sends the other to its partner, which keeps exactly that half (c_s flips between
// partners and no other c_t does: with L = sum c_s X_s over GF(2), c1 = b0^b2, c2 = b1^b2, c3 = b2^b3, c4 = b3 for the
// lane bits b). After min(k, 4) such steps and plain DPP sums for the remaining steps up to 4, every lane holds the
// sums over its 16-lane row of the rows 16 j + m(L), m(L) = sum c_s 2^(s - 1) over the merging steps, and the 16 lanes
// of a row cover every m once. The quarters of the wave (rows of 16 lanes) are summed by the caller. Every lane must
// be active; each partial goes through the same tree of additions whatever its row.
struct FoldLane {
  bool c[4];
  int m;  // the row (mod 16) this lane holds after the merging steps of a fold over n rows
};
__device__ __forceinline__ FoldLane fold_lane(int lane, int n) {
  const int b0 = lane & 1, b1 = (lane >> 1) & 1, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
  FoldLane f;
  f.c[0] = (b0 ^ b2) != 0;
  f.c[1] = (b1 ^ b2) != 0;
  f.c[2] = (b2 ^ b3) != 0;
  f.c[3] = b3 != 0;
  f.m = 0;
#pragma unroll
  for (int s = 0; s < 4; ++s) f.m |= ((1 << (s + 1)) <= n && f.c[s]) ? 1 << s : 0;
  return f;
}
template <int S>  // DPP partner of step S (1..4)
__device__ __forceinline__ float fold_dpp(float v) {
  constexpr int ctrl = S == 1 ? 0xB1 : S == 2 ? 0x4E : S == 3 ? 0x141 : 0x140;
  return DK_DPP_F32(v, ctrl, 0xF);
}
// Merging step S over the half-blocks a (row bit S - 1 clear) and b (set).
template <int S>
__device__ __forceinline__ float fold_merge(float a, float b, bool c) {
  const float keep = c ? b : a, send = c ? a : b;
  return keep + fold_dpp<S>(send);
}
// The merges that become possible once rows [r0, r0 + T) of a fold over N rows are in p: for each step S (ascending),
// every block of 2^S rows that ends inside [r0, r0 + T) merges its two halves into p[block start]. All indices are
// compile-time constants after unrolling.
template <int S, int N, int T>
__device__ __forceinline__ void fold_step(float (&p)[N], int r0, const FoldLane& f) {
  if constexpr ((1 << S) <= N) {
    constexpr int blk = 1 << S, half = blk >> 1;
#pragma unroll
    for (int b = 0; b < N; b += blk) {
      const int end = b + blk - 1;
      if (end >= r0 && end < r0 + T) p[b] = fold_merge<S>(p[b], p[b + half], f.c[S - 1]);
    }
  }
}
template <int N, int T>
__device__ __forceinline__ void fold_rows(float (&p)[N], int r0, const FoldLane& f) {
  fold_step<1, N, T>(p, r0, f);
  fold_step<2, N, T>(p, r0, f);
  fold_step<3, N, T>(p, r0, f);
  fold_step<4, N, T>(p, r0, f);
}
// The plain steps after the merges of a fold over N < 16 rows: the remaining lane bits of the 16-lane row.
template <int N>
__device__ __forceinline__ void fold_finish(float (&p)[N]) {
  if constexpr (N < 2) p[0] += fold_dpp<1>(p[0]);
  if constexpr (N < 4) p[0] += fold_dpp<2>(p[0]);
  if constexpr (N < 8) p[0] += fold_dpp<3>(p[0]);
  if constexpr (N < 16) p[0] += fold_dpp<4>(p[0]);
}

// Same sum, broadcast to every lane (v_readlane of lane 63 into a scalar register).
__device__ __forceinline__ float wave_sum_all(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_lane63(v)), 63));
}

// SwiGLU of one fp16 (gate, up) pair with the reference's rounding points (kernels/fused_swiglu.cu:2,
// reference/ref_ops.py:23-27): silu in fp32 of the fp16 gate, rounded to fp16, then an fp16 product with up.
__device__ __forceinline__ f16 silu_mul(f16 g, f16 u) {
  const float a = (float)g;
  return (f16)(a / (1.0f + expf(-a))) * u;
}

// fp32 dot of two fp16 pairs plus an fp32 accumulator (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// 8 fp16 values of one 16-byte chunk -> fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 h = as_f16x2(v[i]);
    f[2 * i] = (float)h.x;
    f[2 * i + 1] = (float)h.y;
  }
}

// Argmax key of logit v at index i: a 64-bit value whose unsigned order is the argmax ranking (torch.argmax):
// high word 0xFFFFFFFF for NaN, else the float bits made monotonic (negatives inverted, positives with the sign bit
// set, -0 first turned into +0 so the two zeros tie); low word ~i, so that among equal values the lowest index wins.
__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
  uint32_t hi;
  if (v != v) {
    hi = 0xFFFFFFFFu;
  } else {
    const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
    hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)hi << 32) | (uint32_t)~(uint32_t)i;
}

}  // namespace dk
