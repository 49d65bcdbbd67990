// Achievable-read-bandwidth microbenchmark (the role of the reference's bw_read, kernels/gemv_w4a16.cu:133-153):
// a grid-stride sweep of 16-byte loads over a buffer, XOR-folded into one word that is stored only if it equals a
// value it essentially never takes, so the loads cannot be removed and nothing is written in practice.
// Also used read-only to evict the L2 and the MALL between timed iterations.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

template <int UNROLL>
__global__ void __launch_bounds__(1024)
bw_read_kernel(const u32x4* __restrict__ p, size_t n, uint32_t* __restrict__ sink) {
  uint32_t a = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (UNROLL - 1) * stride < n; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) v[k] = load_stream(p + i + k * stride);
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) a ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < n; i += stride) {
    const u32x4 v = load_stream(p + i);
    a ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (a == 0x9e3779b9u) *sink = a;
}

}  // namespace

void launch_bw_read(const void* buf, size_t bytes, void* sink, int blocks, int threads, int unroll, hipStream_t st) {
  const size_t n = bytes / 16;
  if (unroll == 4)
    hipLaunchKernelGGL((bw_read_kernel<4>), dim3(blocks), dim3(threads), 0, st, (const u32x4*)buf, n,
                       (uint32_t*)sink);
  else
    hipLaunchKernelGGL((bw_read_kernel<1>), dim3(blocks), dim3(threads), 0, st, (const u32x4*)buf, n,
                       (uint32_t*)sink);
}

}  // namespace dk
