// HBM read-ceiling probe: what a kernel that only reads reaches on this part, for a given byte count and launch
// shape. It serves the reference's bw_read op (kernels/bindings.cpp:40-43: a read-bandwidth microbenchmark with the
// caller's grid), and it is the known-size read that scales the hardware byte counters.
//
// Design (persistent grid, one contiguous slab per workgroup, checksummed per wave):
//   - the buffer's n 16-byte words are cut into gridDim contiguous slabs of n / G or n / G + 1 words, so every
//     workgroup streams the same number of bytes (to one word) and none waits on a partial last round of another;
//   - a workgroup walks its slab in rounds of DEPTH x blockDim words, double-buffered: a lane issues all DEPTH loads
//     of the next round before it sums the current one (scheduling barriers pin the order), so DEPTH to 2 DEPTH
//     16-byte loads per lane stay in flight; loads past the slab end are clamped to its last word and masked to zero
//     afterwards, so no load sits behind a branch;
//   - the words are summed (mod 2^32); with a sink of at least one slot per wave (sink_words >= gridDim x W, W waves
//     per workgroup) each wave sums over its lanes with DPP and lane 63 stores the wave's sum to sink[b W + w], so the
//     slots add up to the sum of all 32-bit words of the buffer and a caller can check that every byte was read.
//     With a smaller sink (the reference callers pass one word) nothing is written: an empty asm statement takes
//     the sums as inputs, so the loads cannot be dropped, and the kernel ends without a store to wait for (a store
//     of a checksum at the end of each wave cost 0.65 us of a 6 us read of 31.2 MB).
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

__device__ __forceinline__ uint32_t word_sum(u32x4 v) { return (v.x + v.y) + (v.z + v.w); }

#define DK_DPP_U32(v, ctrl, row_mask) \
  ((uint32_t)__builtin_amdgcn_update_dpp(0, (int)(v), (ctrl), (row_mask), 0xF, false))

// Sum over the wave in lane 63 (the u32 twin of wave_sum_lane63; every lane must be active).
__device__ __forceinline__ uint32_t wave_sum_u32_lane63(uint32_t v) {
  v += DK_DPP_U32(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]
  v += DK_DPP_U32(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]
  v += DK_DPP_U32(v, 0x141, 0xF);  // row_half_mirror
  v += DK_DPP_U32(v, 0x140, 0xF);  // row_mirror
  v += DK_DPP_U32(v, 0x142, 0xA);  // row_bcast15, rows 1 and 3
  v += DK_DPP_U32(v, 0x143, 0xC);  // row_bcast31, rows 2 and 3
  return v;
}

// Slab b: `per` words, one more for the first `rem` workgroups; the host passes per, rem and the round counts of both
// slab lengths, so the kernel divides nothing. Rounds are double-buffered: round r + 1's loads are issued before
// round r is summed, so a lane keeps DEPTH to 2 DEPTH loads in flight across round boundaries; a round past the
// slab's end loads its last word (clamped) and sums nothing.
template <int DEPTH>
__device__ __forceinline__ void probe_issue(const u32x4* __restrict__ p, size_t first, size_t T, size_t hi,
                                            u32x4 (&v)[DEPTH]) {
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) v[k] = load_stream(p + min(first + k * T, hi - 1));
}

template <int DEPTH>
__device__ __forceinline__ uint32_t probe_sum(const u32x4 (&v)[DEPTH], size_t first, size_t T, size_t hi) {
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) s += first + k * T < hi ? word_sum(v[k]) : 0u;
  return s;
}

template <int DEPTH>
__global__ void __launch_bounds__(1024)
read_probe_kernel(const u32x4* __restrict__ p, size_t per, uint32_t rem, uint32_t rounds_short,
                  uint32_t rounds_long, uint32_t* __restrict__ sink, uint32_t sink_words) {
  const size_t T = blockDim.x, R = DEPTH * T;
  const uint32_t b = blockIdx.x;
  const bool longer = b < rem;
  const size_t lo = (size_t)b * per + (longer ? b : rem), hi = lo + per + (longer ? 1 : 0);
  const uint32_t rounds = longer ? rounds_long : rounds_short;  // 0 for an empty slab
  uint32_t acc = 0;
  if (rounds > 0) {  // uniform per workgroup
    const size_t f0 = lo + threadIdx.x;
    u32x4 va[DEPTH], vb[DEPTH];
    probe_issue<DEPTH>(p, f0, T, hi, va);
    uint32_t r = 0;
    for (; r + 2 <= rounds; r += 2) {  // whole pairs of rounds, no exit in between (the waits stay partial)
      probe_issue<DEPTH>(p, f0 + (r + 1) * R, T, hi, vb);
      __builtin_amdgcn_sched_barrier(0);
      acc += probe_sum<DEPTH>(va, f0 + r * R, T, hi);
      probe_issue<DEPTH>(p, f0 + (r + 2) * R, T, hi, va);
      __builtin_amdgcn_sched_barrier(0);
      acc += probe_sum<DEPTH>(vb, f0 + (r + 1) * R, T, hi);
    }
    if (r < rounds) acc += probe_sum<DEPTH>(va, f0 + r * R, T, hi);
  }
  const uint32_t waves = blockDim.x >> 6;
  if (sink_words >= gridDim.x * waves) {  // uniform: one slot per wave, the checksum is stored
    acc = wave_sum_u32_lane63(acc);
    if ((threadIdx.x & 63) == 63) sink[b * waves + (threadIdx.x >> 6)] = acc;
  } else {
    asm volatile("" ::"v"(acc));  // the sums are kept (so are the loads), nothing is written
  }
}

template <int DEPTH>
void launch_depth(const void* buf, size_t n, uint32_t* sink, uint32_t sink_words, int blocks, int threads,
                  hipStream_t st) {
  const size_t per = n / (size_t)blocks, R = (size_t)DEPTH * threads;
  hipLaunchKernelGGL((read_probe_kernel<DEPTH>), dim3(blocks), dim3(threads), 0, st, (const u32x4*)buf, per,
                     (uint32_t)(n % (size_t)blocks), (uint32_t)((per + R - 1) / R), (uint32_t)((per + R) / R), sink,
                     sink_words);
}

}  // namespace

void launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, uint32_t sink_words, int blocks, int threads,
                       int depth, hipStream_t st) {
  const size_t n = bytes / 16;
  switch (depth) {
    case 1: launch_depth<1>(buf, n, sink, sink_words, blocks, threads, st); break;
    case 2: launch_depth<2>(buf, n, sink, sink_words, blocks, threads, st); break;
    case 4: launch_depth<4>(buf, n, sink, sink_words, blocks, threads, st); break;
    case 8: launch_depth<8>(buf, n, sink, sink_words, blocks, threads, st); break;
    default: launch_depth<16>(buf, n, sink, sink_words, blocks, threads, st); break;
  }
}

}  // namespace dk
