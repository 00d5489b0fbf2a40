// Diagnostics: plain HBM streaming (read, write, copy) with the access shape the path's
// kernels use (16 bytes per lane, coalesced rows), to measure what this GPU's HBM delivers
// to such loads and stores -- the practical ceiling against which the path's roofline
// fractions are read.  Not part of the delta-rule path.
#include "common.hpp"
#include "rewy_amd.h"

namespace rewy {

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ a, size_t n,
                                                          u32x4* __restrict__ sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) acc ^= a[i];
  // one vector store per work-group keeps the loads live
  if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

__global__ __launch_bounds__(256) void stream_write_kernel(u32x4* __restrict__ a, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    a[i] = u32x4{(uint32_t)i, 1u, 2u, 3u};
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ a, u32x4* __restrict__ b,
                                                          size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) b[i] = a[i];
}

}  // namespace rewy

using namespace rewy;

extern "C" hipError_t fdr_stream_probe(int mode, const void* src, void* dst, long long bytes, int grid,
                                       hipStream_t stream) {
  const int GRID = grid;
  if (bytes <= 0 || bytes % 16 || !dst || (mode != 1 && !src) || grid <= 0 || grid > (1 << 20))
    return hipErrorInvalidValue;
  const size_t n = (size_t)bytes / 16;
  switch (mode) {
    case 0:   // read src; dst receives `grid` 16-byte words
      hipLaunchKernelGGL(stream_read_kernel, dim3(GRID), dim3(256), 0, stream, (const u32x4*)src, n, (u32x4*)dst);
      break;
    case 1:   // write dst
      hipLaunchKernelGGL(stream_write_kernel, dim3(GRID), dim3(256), 0, stream, (u32x4*)dst, n);
      break;
    case 2:   // copy src -> dst
      hipLaunchKernelGGL(stream_copy_kernel, dim3(GRID), dim3(256), 0, stream, (const u32x4*)src, (u32x4*)dst, n);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
