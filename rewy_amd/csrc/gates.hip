// KDA's in-kernel gate activation (use_gate_in_kernel=True) and its backward, as
// the reference documents them (_compat/kda.py:250-294; dA_log / ddt_bias are the
// extra outputs of kda_backward, backends/backward.py:63-73):
//
//   mode 0:  g = -exp(A_log[h]) softplus(x)            x = g_raw + dt_bias[h, k]
//   mode 1:  g = lower_bound sigmoid(exp(A_log[h]) x)
//   mode 2:  g = lower_bound sigmoid(x)                 (no A_log)
//
// Both passes stream [N, H, K] rows once (N = B T tokens, H K columns per token):
// a work-group owns a block of tokens and 2048 columns, a thread 8 consecutive
// columns (16 threads = one head's 128 channels).  The backward also forms
// ddt_bias = sum_n dx and dA_log = sum_{n,k} dx-term per token block into
// partials, summed over the blocks by a second, tiny launch (deterministic, no
// atomics).
#include "common.hpp"

namespace rewy {

constexpr int GT_TOK = 128;        // tokens per work-group
constexpr int GT_COLS = 2048;      // columns per work-group (256 threads x 8)

__device__ __forceinline__ float softplus_f(float x) { return softplus_y(x, exp_f(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return sigmoid_y(exp_f(x)); }

template <bool BF16_IN>
__device__ __forceinline__ void load8(const void* p, size_t off, float (&v)[8]) {
  if constexpr (BF16_IN) {
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

template <bool BF16_OUT>
__device__ __forceinline__ void store8(void* p, size_t off, const float (&v)[8]) {
  if constexpr (BF16_OUT) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = to_bf16(v[e]);
    *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p) + off) = b;
  } else {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + off) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + off + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// g (fp32) from g_raw
template <bool BF16_IN, int MODE>
__global__ __launch_bounds__(256) void kda_gate_fwd_kernel(const void* __restrict__ graw,
                                                           const float* __restrict__ A_log,
                                                           const float* __restrict__ dt_bias, float lower_bound,
                                                           float* __restrict__ g, int N, int HK) {
  const int col = GT_COLS * blockIdx.y + 8 * threadIdx.x;
  if (col >= HK) return;                       // no barriers below
  const int h = col / KD;
  float bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = dt_bias ? dt_bias[col + e] : 0.f;
  const float a = (MODE == 2) ? 1.f : expf(A_log[h]);
  const int n0 = GT_TOK * blockIdx.x, n1 = min(N, n0 + GT_TOK);
  for (int n = n0; n < n1; ++n) {
    const size_t off = (size_t)n * HK + col;
    float x[8], y[8];
    load8<BF16_IN>(graw, off, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xe = x[e] + bias[e];
      if constexpr (MODE == 0) y[e] = -a * softplus_f(xe);
      else y[e] = lower_bound * sigmoid_f(a * xe);
    }
    store8<false>(g, off, y);
  }
}

// dx = dL/dg_raw; partial sums of ddt_bias (per column) and dA_log (per head) per token block
template <bool BF16_IN, int MODE>
__global__ __launch_bounds__(256) void kda_gate_bwd_kernel(const float* __restrict__ dg, const void* __restrict__ graw,
                                                           const float* __restrict__ A_log,
                                                           const float* __restrict__ dt_bias, float lower_bound,
                                                           void* __restrict__ dx, float* __restrict__ part_dt,
                                                           float* __restrict__ part_da, int N, int HK) {
  const int col = GT_COLS * blockIdx.y + 8 * threadIdx.x;
  const bool live = col < HK;                  // whole 16-lane groups (one head) share this
  const int h = live ? col / KD : 0;
  float bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = (live && dt_bias) ? dt_bias[col + e] : 0.f;
  const float a = (MODE == 2 || !live) ? 1.f : expf(A_log[h]);
  float sdt[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float sda = 0.f;
  const int n0 = GT_TOK * blockIdx.x, n1 = min(N, n0 + GT_TOK);
  if (live) {
    for (int n = n0; n < n1; ++n) {
      const size_t off = (size_t)n * HK + col;
      float x[8], d[8], o[8];
      load8<BF16_IN>(graw, off, x);
      load8<false>(dg, off, d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xe = x[e] + bias[e];
        if constexpr (MODE == 0) {
          // g = -a softplus(x): dx = -dg a sigmoid(x), dA_log += dg g
          const float y = exp_f(xe);
          o[e] = -d[e] * a * sigmoid_y(y);
          sda += d[e] * (-a * softplus_y(xe, y));
        } else {
          // g = lb sigmoid(a x): ds = dg lb s (1 - s), dx = ds a, dA_log += ds a x
          const float s = sigmoid_f(a * xe);
          const float ds = d[e] * lower_bound * s * (1.f - s);
          o[e] = ds * a;
          if constexpr (MODE == 1) sda += ds * a * xe;
        }
        sdt[e] += o[e];
      }
      store8<BF16_IN>(dx, off, o);
    }
  }
  if (live) {
    float* pd = part_dt + (size_t)blockIdx.x * HK + col;
    *reinterpret_cast<f32x4*>(pd) = f32x4{sdt[0], sdt[1], sdt[2], sdt[3]};
    *reinterpret_cast<f32x4*>(pd + 4) = f32x4{sdt[4], sdt[5], sdt[6], sdt[7]};
  }
  // a head's 16 lanes -> one dA partial (every lane takes part in the cross-lane sum)
  const float tot = sum_row16(sda);
  if (live && (threadIdx.x & 15) == 0) part_da[(size_t)blockIdx.x * (HK / KD) + h] = tot;
}

// sum the per-block partials: ddt [HK] over nblk_dt rows, dA [H] over nblk_da rows
// Column sums of the per-block partials: ddt[c] = sum_r part_dt[r][c] (HK columns) and
// dA[h] = sum_r sum_{j<G} part_da[r][h G + j] (H G columns).  A work-group takes 16
// columns and splits the rows over 16 slices (four independent accumulators per
// lane, so loads stay in flight), then reduces the slices, and for dA each group of
// G adjacent columns (G divides 16), through LDS.
__global__ __launch_bounds__(256) void kda_gate_sum_kernel(const float* __restrict__ part_dt,
                                                           const float* __restrict__ part_da, float* __restrict__ ddt,
                                                           float* __restrict__ dA, int nrows, int HK, int G) {
  __shared__ float red[16][17];
  __shared__ float tot[16];
  const int H = HK / KD, dt_blocks = ddt ? HK / 16 : 0;
  const bool is_dt = (int)blockIdx.x < dt_blocks;
  const float* src = is_dt ? part_dt : part_da;
  const int cols = is_dt ? HK : H * G;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int c = 16 * (is_dt ? blockIdx.x : blockIdx.x - dt_blocks) + tx;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < cols) {
    int r = ty;
    for (; r + 48 < nrows; r += 64) {
      s0 += src[(size_t)r * cols + c];
      s1 += src[(size_t)(r + 16) * cols + c];
      s2 += src[(size_t)(r + 32) * cols + c];
      s3 += src[(size_t)(r + 48) * cols + c];
    }
    for (; r < nrows; r += 16) s0 += src[(size_t)r * cols + c];
  }
  red[ty][tx] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (ty != 0) return;
  float t = 0.f;
#pragma unroll
  for (int y = 0; y < 16; ++y) t += red[y][tx];
  if (is_dt) {
    if (c < cols) ddt[c] = t;
    return;
  }
  tot[tx] = t;   // read back by lanes of this same wave: LDS operations of a wave stay in order
  if (tx % G == 0 && c < cols) {
    float u = 0.f;
    for (int j = 0; j < G; ++j) u += tot[tx + j];
    dA[c / G] = u;
  }
}

// ddt_bias / dA_log from partials (also used by the chunk kernel's folded gate backward)
hipError_t kda_gate_partials_sum(const float* part_dt, const float* part_da, int nrows, int HK, int G, float* ddt,
                                 float* dA, hipStream_t s) {
  if (!ddt && !dA) return hipSuccess;
  if (G < 1 || 16 % G) return hipErrorInvalidValue;
  const int blocks = (ddt ? HK / 16 : 0) + (dA ? (HK / KD * G + 15) / 16 : 0);
  hipLaunchKernelGGL(kda_gate_sum_kernel, dim3(blocks), dim3(256), 0, s, part_dt, part_da, ddt, dA, nrows, HK, G);
  return hipGetLastError();
}

template <bool BF16_IN>
static hipError_t gate_fwd_launch(int mode, const void* graw, const float* A_log, const float* dt_bias, float lb,
                                  float* g, int N, int HK, hipStream_t s) {
  const dim3 grid((N + GT_TOK - 1) / GT_TOK, (HK + GT_COLS - 1) / GT_COLS);
#define GF(M) hipLaunchKernelGGL((kda_gate_fwd_kernel<BF16_IN, M>), grid, dim3(256), 0, s, graw, A_log, dt_bias, lb, g, N, HK)
  if (mode == 0) GF(0);
  else if (mode == 1) GF(1);
  else GF(2);
#undef GF
  return hipGetLastError();
}

template <bool BF16_IN>
static hipError_t gate_bwd_launch(int mode, const float* dg, const void* graw, const float* A_log,
                                  const float* dt_bias, float lb, void* dx, float* part_dt, float* part_da, int N,
                                  int HK, hipStream_t s) {
  const dim3 grid((N + GT_TOK - 1) / GT_TOK, (HK + GT_COLS - 1) / GT_COLS);
#define GB(M)                                                                                                   \
  hipLaunchKernelGGL((kda_gate_bwd_kernel<BF16_IN, M>), grid, dim3(256), 0, s, dg, graw, A_log, dt_bias, lb, dx, \
                     part_dt, part_da, N, HK)
  if (mode == 0) GB(0);
  else if (mode == 1) GB(1);
  else GB(2);
#undef GB
  return hipGetLastError();
}

}  // namespace rewy

using namespace rewy;

static int gate_mode_of(const float* A_log, int has_lower_bound) {
  if (!has_lower_bound) return A_log ? 0 : -1;
  return A_log ? 1 : 2;
}

extern "C" size_t fdr_kda_gate_workspace_bytes(int B, int T, int H, int K) {
  if (B <= 0 || T <= 0 || H <= 0 || K != KD) return 0;
  const size_t nblk = ((size_t)B * T + GT_TOK - 1) / GT_TOK;
  return nblk * ((size_t)H * KD + H) * sizeof(float);
}

extern "C" hipError_t fdr_kda_gate_fwd(const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
                                       int has_lower_bound, float lower_bound, float* g, int B, int T, int H, int K,
                                       hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0 || K != KD || !g_raw || !g) return hipErrorInvalidValue;
  if ((long long)B * T >= (1LL << 31)) return hipErrorInvalidValue;
  const int mode = gate_mode_of(A_log, has_lower_bound);
  if (mode < 0) return hipErrorInvalidValue;
  const int N = B * T, HK = H * KD;
  return raw_is_bf16 ? gate_fwd_launch<true>(mode, g_raw, A_log, dt_bias, lower_bound, g, N, HK, stream)
                     : gate_fwd_launch<false>(mode, g_raw, A_log, dt_bias, lower_bound, g, N, HK, stream);
}

extern "C" hipError_t fdr_kda_gate_bwd(const float* dg, const void* g_raw, int raw_is_bf16, const float* A_log,
                                       const float* dt_bias, int has_lower_bound, float lower_bound, void* dg_raw,
                                       float* dA_log, float* ddt_bias, void* workspace, int B, int T, int H, int K,
                                       hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0 || K != KD || !dg || !g_raw || !dg_raw || !workspace) return hipErrorInvalidValue;
  if ((long long)B * T >= (1LL << 31)) return hipErrorInvalidValue;
  const int mode = gate_mode_of(A_log, has_lower_bound);
  if (mode < 0) return hipErrorInvalidValue;
  const int N = B * T, HK = H * KD;
  const int nblk = (N + GT_TOK - 1) / GT_TOK;
  float* part_dt = reinterpret_cast<float*>(workspace);
  float* part_da = part_dt + (size_t)nblk * HK;
  hipError_t e = raw_is_bf16 ? gate_bwd_launch<true>(mode, dg, g_raw, A_log, dt_bias, lower_bound, dg_raw, part_dt,
                                                     part_da, N, HK, stream)
                             : gate_bwd_launch<false>(mode, dg, g_raw, A_log, dt_bias, lower_bound, dg_raw, part_dt,
                                                      part_da, N, HK, stream);
  if (e != hipSuccess) return e;
  return kda_gate_partials_sum(part_dt, part_da, nblk, HK, 1, ddt_bias, dA_log, stream);
}

namespace rewy {
// beta = s sigmoid(x) per token and head (use_beta_sigmoid_in_kernel); its backward
// is folded into the chunk kernel's dbeta stores (fdr_chunk_bwd's beta_sigmoid)
template <bool BF16_IN>
__global__ __launch_bounds__(256) void beta_sigmoid_kernel(const void* __restrict__ x, float s,
                                                           float* __restrict__ beta, long long n) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const float xv = BF16_IN ? to_f32(reinterpret_cast<const bf16*>(x)[i]) : reinterpret_cast<const float*>(x)[i];
    beta[i] = s * sigmoid_y(exp_f(xv));
  }
}
}  // namespace rewy

extern "C" hipError_t fdr_beta_sigmoid_fwd(const void* x, int is_bf16, float scale, float* beta, long long n,
                                           hipStream_t stream) {
  if (n <= 0 || !x || !beta || !(scale > 0.f)) return hipErrorInvalidValue;
  const long long blocks = (n + 255) / 256;
  const int grid = (int)(blocks < 8192 ? blocks : 8192);
  if (is_bf16)
    hipLaunchKernelGGL(beta_sigmoid_kernel<true>, dim3(grid), dim3(256), 0, stream, x, scale, beta, n);
  else
    hipLaunchKernelGGL(beta_sigmoid_kernel<false>, dim3(grid), dim3(256), 0, stream, x, scale, beta, n);
  return hipGetLastError();
}
