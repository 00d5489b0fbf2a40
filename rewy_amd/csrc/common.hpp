// Shared device helpers for the gfx950 delta-rule backward kernels.
//
// Operand convention for every MFMA in this library: both operands are held
// "K-contiguous" in LDS, i.e. A as [M][K] and B as [N][K] with the contraction
// index innermost.  One 16-byte read per lane then yields a full 8-element
// fragment of v_mfma_f32_16x16x32_bf16 for either operand.  The accumulator
// layout is the hardware's: lane l holds column (l & 15) and rows
// 4*(l >> 4) + r, r = 0..3, of a 16x16 tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rewy {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int C = 64;     // chunk length
constexpr int KD = 128;   // key width
constexpr int VD = 128;   // value width

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// 8-element fragment of a K-contiguous tile whose row 0 / k 0 is at `base`.
__device__ __forceinline__ bf16x8 frag(const bf16* base, int ld) {
  const int l = lane_id();
  return *reinterpret_cast<const bf16x8*>(base + (l & 15) * ld + 8 * (l >> 4));
}

__device__ __forceinline__ bf16 to_bf16(float x) { return static_cast<bf16>(x); }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

// hi + lo split of an fp32 value into two bf16 (hi exact in bf16, lo the rest).
__device__ __forceinline__ void split_bf16(float x, bf16& hi, bf16& lo) {
  hi = to_bf16(x);
  lo = to_bf16(x - to_f32(hi));
}

__device__ __forceinline__ float fast_exp2(float x) { return exp2f(x); }

// Logical work-group index remapped so that consecutive logical indices stay on
// one XCD (hardware dispatches linear work-group ids round-robin over 8 XCDs,
// each with its own L2).  Identity when the grid is not a multiple of 8.
__device__ __forceinline__ int xcd_logical_block() {
  const int n = gridDim.x;
  const int b = blockIdx.x;
  if (n % 8) return b;
  return (b % 8) * (n / 8) + b / 8;
}

// Sum over the 4 lane groups (lanes l, l^16, l^32, l^48) of a wave.
__device__ __forceinline__ float sum_lane_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Sum over the 16 lanes of one lane group (the 16 columns of a C tile row).
__device__ __forceinline__ float sum_row16(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

}  // namespace rewy
