// Grouped value heads (GVA): the q / k gradients summed over each head's group.
//
// With HV = G H value heads sharing H q / k heads (FLA's head map i_h = i_hv // G), the
// chunk kernels write dq / dk per value head, [rows, H, G, K] bf16 (rows = B T); the
// gradient of q / k is the sum over each group:
//
//   out[r, h, k] = bf16( sum_{j=0..G-1} x[r, h, j, k] )      summed in fp32, j ascending
//
// One pass: every 16-byte piece of the output reads its G input pieces.  Replaces the
// reshape-and-sum the reference leaves to torch after FLA's kernels (a view, an fp32
// copy, a sum and a cast: four passes).  Pieces are walked grid-stride.
#include "common.hpp"
#include "rewy_amd.h"

namespace rewy {

__global__ __launch_bounds__(256) void group_sum_kernel(const bf16* __restrict__ x, bf16* __restrict__ out,
                                                        long long pieces, int G) {
  constexpr int PK = KD / 8;                      // 16-byte pieces per row of K
  for (long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x; p < pieces;
       p += (long long)gridDim.x * blockDim.x) {
    const long long rh = p / PK;                  // (row, head) pair
    const int c8 = 8 * (int)(p % PK);
    const bf16* src = x + (size_t)rh * G * KD + c8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < G; ++j) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(src + (size_t)j * KD);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += to_f32(b[e]);
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf16(acc[e]);
    *reinterpret_cast<bf16x8*>(out + (size_t)rh * KD + c8) = o;
  }
}

}  // namespace rewy

using namespace rewy;

extern "C" hipError_t fdr_group_sum(const void* x, void* out, long long rows, int heads, int group, int K,
                                    hipStream_t stream) {
  if (K != KD || rows < 0 || heads <= 0 || group <= 0 || !x || !out) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  const long long pieces = rows * heads * (KD / 8);
  const long long blocks = (pieces + 255) / 256;
  const int grid = (int)(blocks < 8192 ? blocks : 8192);
  hipLaunchKernelGGL(group_sum_kernel, dim3(grid), dim3(256), 0, stream, (const bf16*)x, (bf16*)out, pieces, group);
  return hipGetLastError();
}
