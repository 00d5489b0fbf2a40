// The two recurrences of the recompute policy in one launch: the reverse state recurrence
// (fdr_state_bwd / fdr_state_bwd_raw_qk) and the forward scan forming u itself
// (fdr_fwd_h_u), which do not depend on each other.  Work-groups [0, n) run the state
// recurrence's body (state_body.hpp) and [n, 2n) the scan's (scan_body.hpp), n = B H V / BV
// each, so the state recurrence's work-groups, the longer chain, are dispatched first.
//
// For batch x heads too small for one recurrence to fill the GPU (n <= 128), the two run
// side by side at twice the tile width each would take alone.  Run as two launches on two
// streams, the fork and join cost ~25 us of host time per backward (two HIP event records
// and stream waits) and two more graph nodes; here they are one launch on the caller's
// stream.  Both bodies are the separate kernels' code, so every output is the same bits.
#include "rewy_amd.h"

#include "scan_body.hpp"
#include "state_body.hpp"

namespace rewy {

struct PairState {
  const bf16* q;        // qg (vector gate, prepared), or the raw q
  const bf16* k;        // kg (vector gate, prepared), or the raw k
  const bf16* w;        // null: formed in-kernel (raw vector gate, FW)
  const float* g;
  const bf16* dO;
  const float* aqk;     // null: formed in-kernel (scalar / no gate, INL); else read
  const float* dht;
  bf16* dh;
  bf16* dr;
  float* dh0;
  const float* beta;    // FW = 1
  const bf16* bgate;    // FW = 2
  const float* akk;     // FW
  int HQ;
};

struct PairScan {
  const bf16* k;        // raw k (HQ heads), or the prepared kg (KGIN, H heads)
  const bf16* v;
  const float* g;
  const float* beta;
  const bf16* bgate;    // u's Z = w_gate v with w given; E = (b k) 2^g with w formed
  const bf16* wgate;
  const float* akk;
  const float* h0;
  bf16* h;
  bf16* vnew;
  float* ht;
  const bf16* w;        // null: formed in-kernel (NOST)
  int HQ;
};

// The XCD-aware map of each half (consecutive logical blocks on one XCD, as
// xcd_logical_block): block b of the launch sits on XCD b % 8, so a half starting at a
// multiple of 8 keeps that pattern.
__device__ __forceinline__ int half_logical(int b, int n) { return n % 8 ? b : (b % 8) * (n / 8) + b / 8; }

template <int BV, int GATE, bool INL, bool RAWQK, int FW, bool VEC_B, bool WG, bool NOST, bool KGIN>
__global__ __launch_bounds__(512) void paired_kernel(PairState s, PairScan f, int n, int T, int H, float scale,
                                                     int vf) {
  __shared__ union {
    StateSmem<BV, GATE, true, INL, FW> st;
    FwdWySmem<BV> sc;
  } sm;
  const int b = blockIdx.x;
  if (b < n) {
    state_bwd_body<BV, GATE, true, 8, false, INL, RAWQK, FW>(sm.st, half_logical(b, n), s.q, s.k, s.w, s.g, s.dO,
                                                               s.aqk, nullptr, s.dht, s.dh, s.dr, s.dh0, T, H, scale,
                                                               nullptr, 0, vf, s.HQ, nullptr, s.beta, s.bgate, s.akk);
  } else {
    fwd_h_wy_body<BV, GATE, VEC_B, false, WG, NOST, KGIN>(sm.sc, half_logical(b - n, n), nullptr, f.k, f.v, f.g,
                                                          f.beta, f.bgate, f.wgate, f.akk, f.h0, nullptr, nullptr,
                                                          nullptr, f.h, f.vnew, f.ht, T, H, nullptr, vf, f.HQ,
                                                          nullptr, f.w);
  }
}

template <int BV, int GATE, bool INL, bool RAWQK, int FW, bool VEC_B, bool WG, bool NOST, bool KGIN>
static hipError_t launch_paired(const PairState& s, const PairScan& f, int B, int T, int H, float scale, int vf,
                                hipStream_t stream) {
  const int n = B * H * (VD / BV);
  hipLaunchKernelGGL((paired_kernel<BV, GATE, INL, RAWQK, FW, VEC_B, WG, NOST, KGIN>), dim3(2 * n), dim3(512), 0,
                     stream, s, f, n, T, H, scale, vf);
  return hipGetLastError();
}

}  // namespace rewy

using namespace rewy;

#define P_ARGS s, f, B, T, H, scale, vf, stream
#define P_BV(...)                                               \
  switch (value_block) {                                        \
    case 16: return launch_paired<16, __VA_ARGS__>(P_ARGS);     \
    case 32: return launch_paired<32, __VA_ARGS__>(P_ARGS);     \
    case 64: return launch_paired<64, __VA_ARGS__>(P_ARGS);     \
    default: return hipErrorInvalidValue;                       \
  }

extern "C" hipError_t fdr_paired_recurrences(
    const void* q, const void* k, const void* w, const void* k_scan, const void* kg, const float* g, int gate_mode,
    const float* beta, const void* b_gate, const void* w_gate, const void* v, const float* Akk, const float* aqk,
    const void* dO, const float* dht, const float* h0, void* dh, void* dr, float* dh0, void* h, void* v_new,
    float* ht, int raw_qk, int state_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk, float scale,
    int value_block, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (value_block != 16 && value_block != 32 && value_block != 64) return hipErrorInvalidValue;
  if (!q || !k || !dO || !dh || !dr || !v || !Akk || !h || !v_new) return hipErrorInvalidValue;
  if (gate_mode < GATE_NONE || gate_mode > GATE_VECTOR || (gate_mode != GATE_NONE && !g)) return hipErrorInvalidValue;
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ) return hipErrorInvalidValue;
  const int vf = state_v_first ? 1 : 0;
  const bool vec_b = w_gate != nullptr;
  if (vec_b ? gate_mode != GATE_VECTOR : !beta) return hipErrorInvalidValue;
  PairState s{(const bf16*)q, (const bf16*)k, (const bf16*)w, g, (const bf16*)dO, aqk, dht, (bf16*)dh, (bf16*)dr,
              dh0, nullptr, nullptr, nullptr, HQ};
  PairScan f{(const bf16*)k_scan, (const bf16*)v, g, beta, (const bf16*)(w ? w_gate : b_gate),
             (const bf16*)w_gate, Akk, h0, (bf16*)h, (bf16*)v_new, ht, (const bf16*)w, HQ};
  if (gate_mode != GATE_VECTOR) {
    // scalar / no gate: raw q / k, w given; Aqk formed by the state recurrence, or read
    if (!w || raw_qk || kg || !k_scan) return hipErrorInvalidValue;
    if (aqk) {
      if (gate_mode == GATE_SCALAR) P_BV(GATE_SCALAR, false, false, 0, false, true, false, false)
      P_BV(GATE_NONE, false, false, 0, false, true, false, false)
    }
    if (gate_mode == GATE_SCALAR) P_BV(GATE_SCALAR, true, false, 0, false, true, false, false)
    P_BV(GATE_NONE, true, false, 0, false, true, false, false)
  }
  if (!aqk) return hipErrorInvalidValue;
  if (!raw_qk) {
    // qg / kg / w as fdr_prepare_wu wrote them (one row per value head); the scan reads that
    // kg (q, k and k_scan's head count is then not used)
    if (!w || !kg) return hipErrorInvalidValue;
    f.k = (const bf16*)kg;
    s.HQ = f.HQ = H;
    if (vec_b) P_BV(GATE_VECTOR, false, false, 0, true, true, false, true)
    P_BV(GATE_VECTOR, false, false, 0, false, true, false, true)
  }
  // raw q / k at 64-wide tiles: qg / kg formed in both recurrences, and w too when null
  if (value_block != 64 || kg || !k_scan) return hipErrorInvalidValue;
  if (w) {
    if (vec_b) return launch_paired<64, GATE_VECTOR, false, true, 0, true, true, false, false>(P_ARGS);
    return launch_paired<64, GATE_VECTOR, false, true, 0, false, true, false, false>(P_ARGS);
  }
  s.akk = Akk;
  if (vec_b) {
    if (!b_gate || HQ != H) return hipErrorInvalidValue;
    s.bgate = (const bf16*)b_gate;
    return launch_paired<64, GATE_VECTOR, false, true, 2, true, false, true, false>(P_ARGS);
  }
  s.beta = beta;
  return launch_paired<64, GATE_VECTOR, false, true, 1, false, false, true, false>(P_ARGS);
}

#undef P_BV
#undef P_ARGS
