// The recompute-policy backward of the scalar-gate / no-gate families (GDN, DeltaNet) as one
// host call: fdr_prepare_wu (w, and Aqk where asked), fdr_paired_recurrences and
// fdr_chunk_bwd, enqueued in that order on one stream with every intermediate carved out of
// one caller-provided workspace.  The three launches are the entry points' own, so every
// output is the bits of the three calls made one by one.  What this saves is host time: for
// small batches the GPU finishes the three kernels in ~26 us, while three foreign-function
// calls, eleven tensor allocations and the per-call argument checks take ~50 us, so the
// eager backward is bound by the host.
#include "rewy_amd.h"

#include <cstdint>

namespace {

constexpr size_t kAlign = 256;

size_t round_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Offsets of the intermediates in the workspace, in order: w, Aqk, dh, dR, h, v_new.
struct Carve {
  size_t off[6];
  size_t total;
  Carve(long long B, long long T, long long H, long long K, long long V, long long chunk) {
    const long long NT = T / chunk;
    const size_t sz[6] = {size_t(B * T * H * K) * 2, size_t(B * T * H * chunk) * 4, size_t(B * NT * H * K * V) * 2,
                          size_t(B * T * H * V) * 2, size_t(B * NT * H * K * V) * 2, size_t(B * T * H * V) * 2};
    total = 0;
    for (int i = 0; i < 6; ++i) {
      off[i] = total;
      total += round_up(sz[i]);
    }
  }
};

}  // namespace

extern "C" size_t fdr_scalar_bwd_workspace_bytes(int B, int T, int H, int K, int V, int chunk) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || chunk <= 0 || T % chunk) return 0;
  return Carve(B, T, H, K, V, chunk).total;
}

extern "C" hipError_t fdr_scalar_bwd(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                     const float* beta, const float* Akk, const void* dO, const float* dht,
                                     const float* h0, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                                     float* dh0, void* workspace, size_t workspace_bytes, float beta_sigmoid,
                                     int aqk_in_prepare, int state_v_first, int B, int T, int H, int qk_heads, int K,
                                     int V, int chunk, float scale, int value_block, hipStream_t stream) {
  // every rule the three entry points would apply to these arguments, checked before the
  // first launch so a rejected call writes nothing
  if (gate_mode != 0 && gate_mode != 1) return hipErrorInvalidValue;
  if ((gate_mode == 1) != (g != nullptr)) return hipErrorInvalidValue;
  if (!q || !k || !v || !beta || !Akk || !dO || !dq || !dk || !dv || !dbeta || !workspace) return hipErrorInvalidValue;
  if (gate_mode == 1 && !dg) return hipErrorInvalidValue;
  if (value_block != 16 && value_block != 32 && value_block != 64) return hipErrorInvalidValue;
  if (B <= 0 || T <= 0 || H <= 0 || qk_heads <= 0 || H % qk_heads || K != 128 || V != 128 || chunk != 64 ||
      T % chunk || !(beta_sigmoid >= 0.f))
    return hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign) return hipErrorInvalidValue;
  const Carve c(B, T, H, K, V, chunk);
  if (workspace_bytes < c.total) return hipErrorInvalidValue;
  char* ws = static_cast<char*>(workspace);
  void* w = ws + c.off[0];
  float* aqk = aqk_in_prepare ? reinterpret_cast<float*>(ws + c.off[1]) : nullptr;
  void* dh = ws + c.off[2];
  void* dr = ws + c.off[3];
  void* h = ws + c.off[4];
  void* v_new = ws + c.off[5];

  hipError_t st = fdr_prepare_wu(aqk ? q : nullptr, k, v, g, gate_mode, beta, nullptr, nullptr, Akk, w, nullptr,
                                 nullptr, nullptr, aqk, B, T, H, qk_heads, K, V, chunk, scale, stream);
  if (st != hipSuccess) return st;
  st = fdr_paired_recurrences(q, k, w, k, nullptr, g, gate_mode, beta, nullptr, nullptr, v, Akk, aqk, dO, dht, h0, dh,
                              dr, dh0, h, v_new, nullptr, 0, state_v_first, B, T, H, qk_heads, K, V, chunk, scale,
                              value_block, stream);
  if (st != hipSuccess) return st;
  return fdr_chunk_bwd(q, k, v, v_new, dO, dr, g, gate_mode, beta, nullptr, nullptr, Akk, h, dh, dq, dk, dv, dg,
                       dbeta, beta_sigmoid, nullptr, nullptr, 0, B, T, H, qk_heads, K, V, chunk, scale, stream);
}
