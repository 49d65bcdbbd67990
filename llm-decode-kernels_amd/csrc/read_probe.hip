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
//   - each wave sums its words (mod 2^32) with DPP and lane 63 stores the wave's sum to sink[(b W + w) mod sink_words]
//     (W waves per workgroup): no LDS and no barrier, every wave retires on its own. With sink_words >= gridDim x W
//     every wave has its own slot and the slots add up to the sum of all 32-bit words of the buffer, so a caller can
//     check that every byte was read; with fewer slots a slot holds the sum of one of the waves that map to it.
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

// Slab b: `per` words, one more for the first `rem` workgroups (per = n / G, rem = n % G from the host, so the kernel
// divides nothing). Rounds are double-buffered: round r + 1's loads are issued before round r is summed, so a lane
// keeps DEPTH to 2 DEPTH loads in flight across round boundaries; a round past the slab's end loads its last word
// (clamped) and sums nothing.
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
read_probe_kernel(const u32x4* __restrict__ p, size_t per, uint32_t rem, uint32_t* __restrict__ sink,
                  uint32_t sink_words) {
  const size_t T = blockDim.x, R = DEPTH * T;
  const uint32_t b = blockIdx.x;
  const size_t lo = (size_t)b * per + min(b, rem), hi = lo + per + (b < rem ? 1 : 0);
  uint32_t acc = 0;
  if (lo < hi) {  // uniform per workgroup (an empty slab reads nothing)
    const size_t rounds = (hi - lo + R - 1) / R, f0 = lo + threadIdx.x;
    u32x4 va[DEPTH], vb[DEPTH];
    probe_issue<DEPTH>(p, f0, T, hi, va);
    size_t r = 0;
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
  acc = wave_sum_u32_lane63(acc);
  if ((threadIdx.x & 63) == 63) {
    const uint32_t slot = (b * (blockDim.x >> 6) + (threadIdx.x >> 6)) % sink_words;  // < 2^28: no overflow
    __hip_atomic_store(sink + slot, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int DEPTH>
void launch_depth(const void* buf, size_t n, uint32_t* sink, uint32_t sink_words, int blocks, int threads,
                  hipStream_t st) {
  hipLaunchKernelGGL((read_probe_kernel<DEPTH>), dim3(blocks), dim3(threads), 0, st, (const u32x4*)buf,
                     n / (size_t)blocks, (uint32_t)(n % (size_t)blocks), sink, sink_words);
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
