// L2 normalisation of q / k over the key dimension (use_qk_l2norm_in_kernel=True,
// reference _compat/kda.py:202-206 and FLA's l2norm_fwd / l2norm_bwd), forward and
// backward, one pass each:
//
//   forward:   r = (sum_k x^2 + eps)^-1/2,  y = x r                    (y in x's dtype, r fp32)
//   backward:  dx = r (dy - y (y . dy)),     y = x r recomputed in fp32
//
// A row is 128 channels: 16 lanes x 8 channels, four rows per wave instruction; the
// row sums run across the 16 lanes (DPP).  Rows are walked grid-stride.
#include "common.hpp"

namespace rewy {

template <bool BF16>
__device__ __forceinline__ void ld8(const void* p, size_t off, float (&v)[8]) {
  if constexpr (BF16) {
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p) + off);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_f32(b[e]);
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + off);
    const f32x4 c = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + off + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[e + 4] = c[e];
    }
  }
}

template <bool BF16>
__device__ __forceinline__ void st8(void* p, size_t off, const float (&v)[8]) {
  if constexpr (BF16) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = to_bf16(v[e]);
    *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p) + off) = b;
  } else {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + off) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + off + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// Every lane runs the same trip count (rows beyond the end are clamped and not
// stored), so the cross-lane sums see all 16 lanes of a row.
template <bool BF16>
__global__ __launch_bounds__(256) void l2norm_fwd_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                         float* __restrict__ rstd, long long rows, float eps) {
  const long long per_iter = (long long)gridDim.x * 16;
  const int sub = threadIdx.x >> 4, c8 = 8 * (threadIdx.x & 15);
  for (long long r0 = (long long)blockIdx.x * 16; r0 < rows; r0 += per_iter) {
    const long long row = r0 + sub;
    const bool live = row < rows;
    const size_t off = (size_t)(live ? row : rows - 1) * KD + c8;
    float v[8];
    ld8<BF16>(x, off, v);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[e] * v[e];
    s = sum_row16(s);
    const float r = 1.f / sqrtf(s + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= r;
    if (live) {
      st8<BF16>(y, off, v);
      if ((threadIdx.x & 15) == 0 && rstd) rstd[row] = r;
    }
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const void* __restrict__ x, const float* __restrict__ rstd,
                                                         const void* __restrict__ dy, void* __restrict__ dx,
                                                         long long rows) {
  const long long per_iter = (long long)gridDim.x * 16;
  const int sub = threadIdx.x >> 4, c8 = 8 * (threadIdx.x & 15);
  for (long long r0 = (long long)blockIdx.x * 16; r0 < rows; r0 += per_iter) {
    const long long row = r0 + sub;
    const bool live = row < rows;
    const long long rr = live ? row : rows - 1;
    const size_t off = (size_t)rr * KD + c8;
    float v[8], d[8];
    ld8<BF16>(x, off, v);
    ld8<BF16>(dy, off, d);
    const float r = rstd[rr];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] *= r;                                  // y in fp32
      s += v[e] * d[e];
    }
    s = sum_row16(s);
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = r * (d[e] - v[e] * s);
    if (live) st8<BF16>(dx, off, d);
  }
}

static unsigned norm_grid(long long rows) {
  const long long blocks = (rows + 15) / 16;
  return (unsigned)(blocks < 8192 ? blocks : 8192);
}

}  // namespace rewy

using namespace rewy;

extern "C" hipError_t fdr_l2norm_fwd(const void* x, int is_bf16, void* y, float* rstd, long long rows, int K,
                                     float eps, hipStream_t stream) {
  if (!x || !y || rows <= 0 || K != KD) return hipErrorInvalidValue;
  if (is_bf16)
    hipLaunchKernelGGL(l2norm_fwd_kernel<true>, dim3(norm_grid(rows)), dim3(256), 0, stream, x, y, rstd, rows, eps);
  else
    hipLaunchKernelGGL(l2norm_fwd_kernel<false>, dim3(norm_grid(rows)), dim3(256), 0, stream, x, y, rstd, rows, eps);
  return hipGetLastError();
}

extern "C" hipError_t fdr_l2norm_bwd(const void* x, int is_bf16, const float* rstd, const void* dy, void* dx,
                                     long long rows, int K, hipStream_t stream) {
  if (!x || !rstd || !dy || !dx || rows <= 0 || K != KD) return hipErrorInvalidValue;
  if (is_bf16)
    hipLaunchKernelGGL(l2norm_bwd_kernel<true>, dim3(norm_grid(rows)), dim3(256), 0, stream, x, rstd, dy, dx, rows);
  else
    hipLaunchKernelGGL(l2norm_bwd_kernel<false>, dim3(norm_grid(rows)), dim3(256), 0, stream, x, rstd, dy, dx, rows);
  return hipGetLastError();
}
