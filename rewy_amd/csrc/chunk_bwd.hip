// Chunk-parallel part of the delta-rule backward: residual-WY local products,
// matrix intra (KDA/GDN2 vector gates, Gram-free scalar-gate form for GDN and
// DeltaNet), state-gradient epilogue and the in-chunk reverse gate cumsum, fused
// per (chunk, head): one work-group per chunk-head (KDA, GDN2), or one persistent
// work-group per CU that walks chunk-heads with direct HBM -> LDS prefetch
// (scalar / no gate).
//
// Replaces, for one 64-token chunk of one head, the reference's
//   residual_tri_beta_producer        kernels/kda_residual_tri_beta.py:8-73
//   residual_wy_local_beta_consumer   kernels/kda_residual_local_beta_consumer.py:23-180
//   endpoint_matrix_kernel            kernels/endpoint_intra.py:16-297
//   residual_scalar.producer (VECTOR) kernels/residual_scalar.py:11-43
//   joint_consumer                    kernels/gdn2_consumer_fp32.py:8-75
//   scalar_liveness_gpu.unified       kernels/scalar_liveness_gpu.py:12-84
// plus the dAqk half of FLA's chunk_kda_bwd_dAv and FLA's reverse chunk-local
// cumsum of dg.  With h the state at the chunk start, dh the state gradient at
// the chunk end, R = v_new, A = Akk and gates in log2 units:
//
//   P  = A^T dR                 (residual product 1)
//   D  = -strict_tril(P R^T)    (residual product 2)
//   Eb = -P h^T                 (residual product 3: direct gradient of E = b k exp2(g))
//   L  = scale tril(dO R^T)     (dAqk)
//   dq = scale (dO h^T) exp2(g)             + uq
//   dk = (R dh^T) exp2(g_last - g) + b exp2(g) Eb + b ue + uk
//   uq = sum_{s<=i} L_is k_s 2^(g_i-g_s),  ue = sum_{s<i} D_is k_s 2^(g_i-g_s)
//   uk = sum_{s>=i} (L_si q_s + D_si b_s k_s) 2^(g_s-g_i)
//   dG = q dq - k dks + b k exp2(g) Eb + k (b ue - uk)  (+ last-row state terms)
//   dg = reverse_cumsum(dG)
//
// Vector gates: per column and 16-row block, 2^(g_i-g_s) = ET_i 2^(top_I - bot_J) EB_s
// with ET = 2^(g - top) <= 1 and EB = 2^(bot - g) <= 1 taken at the blocks' gate
// extremes; a diagonal block whose gate span reaches 80 (log2 units) is evaluated
// pairwise instead, the reference's safety rule (endpoint_intra.py:98-102).  Scalar gates are
// applied exactly to the 64x64 L and D tiles, so no Gram matrix is formed and
// no anchor is needed.  The intra operands are split into bf16 hi + lo so each
// contraction runs as three bf16 MFMAs with fp32 accumulation (the reference
// uses tf32x3 dots for these).
//
// Work split over 8 waves: in phase 1 wave (cs, th) owns the value rows
// [32 cs, 32 cs + 32) and the token tiles th and 2 + th of P^T; in phase 2 each wave
// computes two 16 x 16 tile pairs of L and D; from phase 3 on wave w owns the 16 key
// columns [16 w, 16 w + 16) over all 64 rows.
// Token-major inputs sit in LDS row-major as in HBM (XOR-swizzled 16-byte chunks);
// contractions over tokens read them transposed (ds_read_b64_tr_b16).  P and the
// L/D tiles are produced by MFMAs whose accumulator layout stores contiguously
// into the orientation the next contraction reads.
#include <atomic>

#include "common.hpp"
#include "rewy_amd.h"

namespace rewy {

enum GateModeC { CG_NONE = 0, CG_SCALAR = 1, CG_VECTOR = 2 };

// Persistent, prefetching chunk kernel for the scalar / no-gate families (1), also
// for KDA (2), or never (0, the default).  It had taken GDN's chunk kernel from 0.57 to
// 0.44 ms when the one-work-group-per-chunk-head form waited for every load at each barrier;
// since that form's LDS-only barriers and heads-fastest item order it is the faster one for
// every family and size measured (GDN B=8 T=4096 H=16 chunk kernel 442 vs 449 us, B=1 T=2048
// H=16 DeltaNet backward 116 vs 120 us under graph replay): kept as a build option for A/B.
#ifndef REWY_CHUNK_PIPE
#define REWY_CHUNK_PIPE 0
#endif

namespace post {
constexpr int LDT = 72;    // bf16 pitch of [.][64] tiles
constexpr int T64 = C * LDT * 2;     // bytes of one [64][72] bf16 tile
constexpr int T128 = KD * LDT * 2;   // bytes of one [128][72] bf16 tile
}  // namespace post

template <int GATE, bool VEC_B, bool INTRA = false, bool PIPE = false, bool ORIG = false>
struct PostLayout {
  // PIPE (persistent kernel): dR, R, dO sit in a separate buffer X filled by
  // direct HBM -> LDS copies while the previous chunk-head finishes, and q, k, g
  // are copied the same way into region B at the start of the chunk-head.
  // region A.  phases 0-1: A hi/lo [t][s] (and, unpipelined, dR swizzled).
  //            phases 2+:  L, D row-major hi/lo, and (GDN2) L^T, D^T hi/lo.
  // GDN2 keeps explicit L^T / D^T copies (measured faster for its register budget);
  // the other families read L^T / D^T transposed from L / D.
  static constexpr bool LT_COPY = GATE == CG_VECTOR && VEC_B && !INTRA;
  static constexpr int TQ = C * KD * 2;   // bytes of one swizzled [64][128] bf16 tile
  static constexpr int OFF_AKTH = 0, OFF_AKTL = C * C * 2, OFF_DRT = 2 * C * C * 2;
  static constexpr int OFF_LRH = 0, OFF_LRL = post::T64, OFF_DRH = 2 * post::T64, OFF_DRL = 3 * post::T64;
  static constexpr int OFF_LTH = 4 * post::T64, OFF_LTL = 5 * post::T64, OFF_DTH = 6 * post::T64,
                       OFF_DTL = 7 * post::T64;
  static constexpr int A1 = 2 * C * C * 2 + (PIPE ? 0 : TQ);
  static constexpr int A2 = (LT_COPY ? 8 : 4) * post::T64;
  static constexpr int REGION_A = A1 > A2 ? A1 : A2;
  // region B (offsets from its start).  Unpipelined, phases 0-3: P, R, dO swizzled.
  // Phases 3+ (from phase 0 when pipelined): q, k (, b) swizzled, vector g (fp32, g_off).
  static constexpr int OFF_P = 0, OFF_R = TQ, OFF_DO = 2 * TQ;
  static constexpr int GT_BYTES = GATE == CG_VECTOR ? C * KD * 4 : 0;
  static constexpr int OFF_QT = 0, OFF_KT = TQ, OFF_GT = 2 * TQ;
  static constexpr int OFF_BT = OFF_GT + GT_BYTES;
  static constexpr int B1 = PIPE ? 0 : 3 * TQ;
  // (pipelined: g in an array of its own)
  static constexpr int B2 = 2 * TQ + (PIPE ? 0 : GT_BYTES) + (VEC_B ? TQ : 0);
  static constexpr int REGION_B = B1 > B2 ? B1 : B2;
  // small per-row arrays (floats)
  // S_FB (scalar beta): the direct dbeta terms of |beta| < 1e-6 rows as per-wave partials,
  // [8][64] from phase 1 (one per column strip and value tile) then [8][64] from phase 5,
  // summed in a fixed order (no LDS atomics: the result does not depend on wave timing)
  static constexpr int S_BETA = 0, S_G = 64, S_DBA = 128, S_DG = 448, S_GL = 960, S_ANY = 1088, S_FB = 1096,
                       S_N = S_FB + (VEC_B ? 0 : 16 * 64);
  static constexpr int SMALL = S_N * 4;
  static constexpr int X_BYTES = PIPE ? 3 * TQ + GT_BYTES : 0;
  // the original formulation's extra tiles: Z = beta v, E = beta k 2^g, W-bar (bf16 [64][128]);
  // later T hi/lo over Z and J hi/lo over E ([64][64] each)
  static constexpr int O_BYTES = ORIG ? 3 * TQ : 0;
  static constexpr int OFF_O = REGION_A + REGION_B + SMALL;
  static constexpr int BYTES = REGION_A + REGION_B + SMALL + X_BYTES + O_BYTES;
  static constexpr bool FITS = BYTES <= 160 * 1024;
  static_assert(PIPE || FITS, "LDS budget");
};

// fp32 gate tile [64][128] without padding: the 16-byte chunk c of row r sits at
// chunk c ^ 4 ((r >> 2) & 3), so the 4 rows 4 apart that one read of 16
// consecutive columns touches fall on distinct banks.
__device__ __forceinline__ int g_off(int r, int col) {
  return r * KD + ((((col >> 2) ^ (((r >> 2) & 3) << 2))) << 2) + (col & 3);
}

// Work-group barrier for LDS only, written as one asm block: the persistent
// kernel keeps direct-to-LDS copies in flight across barriers on purpose (each
// copy is waited for explicitly, with vmcnt, before the barrier that publishes it).
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Position of one (batch, chunk, head) work item in the T-major tensors.  Heads
// run fastest: work-groups in flight together read neighbouring heads of the
// same tokens, i.e. contiguous HBM rows.
// With cu_seqlens / chunk_indices (a packed variable-length batch: B = 1, T = 64 x the
// chunk count) the chunk's first token and row count come from them; n = 64 otherwise.
struct ChunkItem {
  int h, c, b, n;
  size_t tok0, kofs, vofs, hoff, aofs;
  __device__ __forceinline__ ChunkItem(int item, int T, int H, const int* cu = nullptr, const int* ci = nullptr) {
    const int NT = T / C;
    h = item % H;
    c = (item / H) % NT;
    b = item / (H * NT);
    n = C;
    tok0 = (size_t)b * T + (size_t)c * C;
    if (cu) {
      const Rows<true> r = chunk_rows<true>(cu, ci, b, c, T);
      tok0 = r.tok0;
      n = r.n;
    }
    kofs = tok0 * H * KD + (size_t)h * KD;
    vofs = tok0 * H * VD + (size_t)h * VD;
    hoff = (((size_t)b * NT + c) * H + h) * KD * VD;
    aofs = (tok0 * H + h) * C;
  }
};

// Per-thread inputs of phase 0 that the persistent kernel fetches one item
// ahead: A (fp32, [t][s] rows of 64; two 16-byte pieces, lanes along rows), and
// beta, the scalar gate of row tid & 63 and the last-row gate of column tid & 127.
// Loaded by every thread (clamped rows) so that no branch splits the vmcnt count.
struct PhaseIn {
  f32x4 a[2];
  float beta, g, gl;
};

template <int GATE, bool VEC_B, bool MAP = false>
__device__ __forceinline__ void load_phase_in(const float* __restrict__ akk, const float* __restrict__ beta,
                                              const float* __restrict__ g, const ChunkItem& it, int H, int tid,
                                              PhaseIn& pin) {
  const Rows<MAP> rw{it.tok0, it.n};
  const size_t rsa = (size_t)H * C;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    pin.a[i] = *reinterpret_cast<const f32x4*>(
        tril_src(rw.src(akk + it.aofs + (size_t)(p >> 4) * rsa + 4 * (p & 15), p >> 4), p >> 4, p & 15));
  }
  const int t = tid & (C - 1);
  const size_t row = (it.tok0 + t) * H + it.h;
  pin.beta = 0.f;
  pin.g = 0.f;
  pin.gl = 0.f;
  if constexpr (!VEC_B) pin.beta = *rw.src(beta + row, t);
  if constexpr (GATE == CG_SCALAR) {
    pin.g = g[(it.tok0 + rw.clamp(t)) * H + it.h];
    pin.gl = g[(it.tok0 + rw.clamp(C - 1)) * H + it.h];
  } else if constexpr (GATE == CG_VECTOR) {
    pin.gl = g[it.kofs + (size_t)rw.clamp(C - 1) * H * KD + (tid & (KD - 1))];
  }
}

// A hi/lo into the [t][s] tiles read transposed by phase 1
__device__ __forceinline__ void stage_akk(const PhaseIn& pin, bf16* sAh, bf16* sAl, int tid) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, ch = p & 15;
    bf16x4 lo;
    const bf16x4 hi = split_hi4(tril_piece(pin.a[i], t, ch), lo);
    *reinterpret_cast<bf16x4*>(sAh + tr_off<8>(t, 4 * ch)) = hi;
    *reinterpret_cast<bf16x4*>(sAl + tr_off<8>(t, 4 * ch)) = lo;
  }
}

// s_waitcnt immediate for vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// q, k of one item into swizzled [64][128] tiles, vector g into the g_off tile
template <int GATE>
__device__ __forceinline__ void dma_qkg(bf16* sQ, bf16* sK, float* sGr, const bf16* __restrict__ q,
                                        const bf16* __restrict__ k, const float* __restrict__ g,
                                        const ChunkItem& it, int H, int HQ, int tid) {
  const size_t rsk = (size_t)H * KD;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
  const QKRows qr = qk_rows(it.tok0, it.h, H, HQ);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    dma_rows4(sQ, 8 * w + 4 * j, q + qr.ofs, qr.rs, l);
    dma_rows4(sK, 8 * w + 4 * j, k + qr.ofs, qr.rs, l);
  }
  if constexpr (GATE == CG_VECTOR) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {       // 2 rows of 512 bytes per instruction
      const int r0 = 8 * w + 2 * j, r = r0 + (l >> 5), pc = l & 31;
      const float* src = g + it.kofs + (size_t)r * rsk + 4 * (pc ^ (((r >> 2) & 3) << 2));
      dma16(src, sGr + r0 * KD);
    }
  }
}

// dR, R = v_new and dO of one item into the swizzled [64][128] tiles x[0..2]:
// wave w copies rows 8 w .. 8 w + 7 of each
__device__ __forceinline__ void dma_x(bf16* xbuf, const bf16* __restrict__ dR, const bf16* __restrict__ vnew,
                                      const bf16* __restrict__ dO, const ChunkItem& it, int H, int tid) {
  const size_t rsv = (size_t)H * VD;
  const int r0 = 8 * __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    dma_rows4(xbuf, r0 + 4 * j, dR + it.vofs, rsv, l);
    dma_rows4(xbuf + C * KD, r0 + 4 * j, vnew + it.vofs, rsv, l);
    dma_rows4(xbuf + 2 * C * KD, r0 + 4 * j, dO + it.vofs, rsv, l);
  }
}

// KDA's in-kernel gate backward folded into the dg stores (use_gate_in_kernel): the
// activation's gradient is applied to dg where it is formed, and ddt_bias / dA_log
// partials are written per (batch, chunk) instead of the fp32 dg.
struct GateFoldArgs {
  const void* graw;      // raw gate input [B,T,H,K], fp32 or bf16
  const float* A_log;    // [H] or null (lower_bound form without A_log)
  const float* dt_bias;  // [H*K] or null
  float lower_bound;
  void* dx;              // dL/dg_raw, g_raw's dtype
  float* part_dt;        // [B*NT][H*K]: sum over a chunk's rows of dx
  float* part_da;        // [B*NT][H][8]: dA_log terms per chunk, head and column strip
};

// The body serves two kernels: the full chunk backward (INTRA = false) and the
// standalone matrix intra (INTRA = true: L and D are given, the partial dq, dk,
// dg, db are read-modify-written in fp32, no state terms and no cumsum).
// FOLD >= 0: the gate backward is folded in, bf16 g_raw if FOLD & 1, activation FOLD >> 1:
// 0: -exp(A) softplus(x), 1: lb sigmoid(exp(A) x), 2: lb sigmoid(x).
// HVF: the per-chunk states h are [V,K] (FLA's state_v_first layout) instead of [K,V].
// ORIG (KDA, comparator only): the local WY backward in the original 7-product formulation
// (W-bar = -dR h^T, E-bar = A^T W-bar, Z-bar = A^T dR, T = dR Z^T + W-bar E^T, J = A^T T,
// D = -strict_tril(J A^T); dbeta by its direct VJP on every row) in place of the residual
// triple (P = A^T dR, D = -strict_tril(P R^T), E-bar = -P h^T).
// MAP: a packed variable-length batch whose sequences start anywhere (cu, ci: cu_seqlens and
// chunk_indices); a sequence's last chunk may hold fewer than 64 rows, whose missing rows
// read as zeros (the gate cumsum's as its last row) and are never written.
// WY (KDA): the kernel-level WY seam alone -- every term but the matrix intra, dq / dk in fp32
// (dq32, dk32), dg before the in-chunk reverse cumsum, dbeta complete for |beta| >= 1e-6 rows
// (the direct terms otherwise), and dA = D, the gradient the intra consumes as dAkk.
template <int GATE, bool VEC_B, bool INTRA, bool PIPE = false, int FOLD = -1, bool HVF = false, bool ORIG = false,
          bool MAP = false, bool WY = false>
__device__ __forceinline__ void chunk_body(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const bf16* __restrict__ hst,
    const bf16* __restrict__ dhst, bf16* __restrict__ dq_out, bf16* __restrict__ dk_out,
    bf16* __restrict__ dv_out, float* __restrict__ dg_out, float* __restrict__ dbeta_out,
    bf16* __restrict__ db_out, bf16* __restrict__ dw_out, int T, int H, float scale,
    const float* __restrict__ daqk, float* __restrict__ dq32, float* __restrict__ dk32,
    float* __restrict__ db32, int beta_complete, int item, int next_item, char* regA, char* regB,
    float* small, bf16* xbuf, float* gbuf, PhaseIn& pin, const GateFoldArgs* gf = nullptr,
    float beta_sig = 0.f, int HQ = 0, const int* cu = nullptr, const int* ci = nullptr, float* dA_wy = nullptr) {
  if (HQ <= 0) HQ = H;
  using LY = PostLayout<GATE, VEC_B, INTRA, PIPE, ORIG>;
  static_assert(!ORIG || (GATE == CG_VECTOR && !VEC_B && !INTRA && !PIPE), "original formulation: KDA only");
  static_assert(!MAP || (!PIPE && !ORIG), "variable-length rows: the plain, gate-fold, intra and WY kernels");
  static_assert(!WY || (GATE == CG_VECTOR && !INTRA && !PIPE && !ORIG && FOLD < 0),
                "the WY seam: KDA and GDN2");
  using post::LDT;
  auto B16 = [&](int off) { return reinterpret_cast<bf16*>(regA + off); };
  auto B16b = [&](int off) { return reinterpret_cast<bf16*>(regB + off); };
  bf16* sAh = B16(LY::OFF_AKTH);    // A rows [s][t], hi
  bf16* sAl = B16(LY::OFF_AKTL);    // A rows, lo
  // dR, R, dO rows [t][v], swizzled: the persistent kernel's prefetch buffer, or staged here
  bf16* sdR = PIPE ? xbuf : B16(LY::OFF_DRT);
  bf16* sR = PIPE ? xbuf + C * KD : B16b(LY::OFF_R);
  bf16* sdO = PIPE ? xbuf + 2 * C * KD : B16b(LY::OFF_DO);
  // P rows [t][v], swizzled: over dR once phase 1 has read it (persistent kernel)
  bf16* sP = PIPE ? xbuf : B16b(LY::OFF_P);
  bf16* Lrh = B16(LY::OFF_LRH);
  bf16* Lrl = B16(LY::OFF_LRL);
  bf16* Drh = B16(LY::OFF_DRH);
  bf16* Drl = B16(LY::OFF_DRL);
  bf16* Lth = B16(LY::OFF_LTH);
  bf16* Ltl = B16(LY::OFF_LTL);
  bf16* Dth = B16(LY::OFF_DTH);
  bf16* Dtl = B16(LY::OFF_DTL);
  bf16* sQ = B16b(LY::OFF_QT);      // q rows [t][k] (swizzled)
  bf16* sK = B16b(LY::OFF_KT);      // k rows
  float* sGr = PIPE ? gbuf : reinterpret_cast<float*>(regB + LY::OFF_GT);   // g rows [t][k] (g_off)
  bf16* sB = B16b(LY::OFF_BT);      // erase-gate rows (GDN2)
  float* sBeta = small + LY::S_BETA;   // scalar beta per row
  float* sG = small + LY::S_G;         // scalar gate per row (log2)
  float* sDbA = small + LY::S_DBA;     // [4][64] sum_v P R per column strip (beta != 0 rows)
  float* sFb = small + LY::S_FB;       // direct dbeta terms (beta ~ 0 rows), per-wave partials
  float* sDg = small + LY::S_DG;       // [8][64] scalar gate: dG row sums per wave
  float* sGl = small + LY::S_GL;       // [128] last-row gate (log2) per column
  int* sAny = reinterpret_cast<int*>(small + LY::S_ANY);   // [8] per-wave "some beta ~ 0" flags

  const ChunkItem pos = MAP ? ChunkItem(item, T, H, cu, ci) : ChunkItem(item, T, H);
  const Rows<MAP> rw{pos.tok0, pos.n};
  const int h = pos.h;
  // the lane index is made opaque per call so that a persistent caller's loop
  // cannot hoist the (loop-invariant) LDS address arithmetic out of the body
  int tid_o = threadIdx.x;
  asm volatile("" : "+v"(tid_o));
  const int tid = tid_o, l = tid_o & 63, wv = __builtin_amdgcn_readfirstlane(tid_o >> 6);
  const int cs = wv & 3;          // column strip: k (or v) in [32 cs, 32 cs + 32)
  const int th = wv >> 2;         // phase 1: token tiles th and 2 + th
  const int lc = l & 15, lg = l >> 4;
  const size_t tok0 = pos.tok0;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD, rsa = (size_t)H * C;
  const size_t hoff = pos.hoff;
  const size_t kofs = pos.kofs;    // [t][k] tensors of this chunk-head
  const size_t vofs = pos.vofs;    // [t][v] tensors
  const bf16* vb = v + vofs;
  const int kk = 16 * wv + lc;                 // this lane's key column from phase 3 on
  // state tiles for phase 3: wave wv owns key columns [16 wv, 16 wv + 16).  The
  // persistent kernel loads them first, ahead of this item's q, k, g copies.
  bf16x8 fh[4], fdh[4];
  auto load_state = [&]() {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const size_t o = hoff + (size_t)kk * VD + 32 * ks + 8 * lg;
      if constexpr (HVF) {
        // h[v][k]: the 8 values of column kk this lane needs are KD apart
#pragma unroll
        for (int j = 0; j < 8; ++j) fh[ks][j] = hst[hoff + (size_t)(32 * ks + 8 * lg + j) * KD + kk];
      } else {
        fh[ks] = *reinterpret_cast<const bf16x8*>(hst + o);
      }
      fdh[ks] = *reinterpret_cast<const bf16x8*>(dhst + o);
    }
  };
  if constexpr (PIPE) load_state();

  // ---------------- phase 0: stage A (hi/lo), dR, R, dO row-major; beta, gates ----------------
  int any_fb = 0;
  if constexpr (INTRA) {
    // L = tril(dAqk) (diagonal included), D = strict_tril(dAkk), split hi/lo, row-major
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;        // 1024 pieces of 4 fp32: row p >> 4
      const int row = p >> 4, c4 = (p & 15) * 4;
      // (a packed batch's missing rows read as zeros; their columns lie above the diagonal
      // of every row that exists)
      f32x4 a = *reinterpret_cast<const f32x4*>(rw.src(daqk + (tok0 * H + h) * C + (size_t)row * rsa + c4, row));
      f32x4 d = *reinterpret_cast<const f32x4*>(rw.src(akk + (tok0 * H + h) * C + (size_t)row * rsa + c4, row));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (c4 + j > row) a[j] = 0.f;
        if (c4 + j >= row) d[j] = 0.f;
      }
      bf16x4 lo;
      bf16x4 hi = split_hi4(a, lo);
      *reinterpret_cast<bf16x4*>(Lrh + row * LDT + c4) = hi;
      *reinterpret_cast<bf16x4*>(Lrl + row * LDT + c4) = lo;
      hi = split_hi4(d, lo);
      *reinterpret_cast<bf16x4*>(Drh + row * LDT + c4) = hi;
      *reinterpret_cast<bf16x4*>(Drl + row * LDT + c4) = lo;
    }
    if (tid < C) {
      if constexpr (!VEC_B) sBeta[tid] = *rw.src(beta + (tok0 + tid) * H + h, tid);
    }
  } else {
    // (the persistent kernel stages A hi/lo at the end of the previous item)
    if constexpr (!PIPE) {
      load_phase_in<GATE, VEC_B, MAP>(akk, beta, g, pos, H, tid, pin);
      stage_akk(pin, sAh, sAl, tid);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;        // 1024 16-byte pieces per tile; lanes run along rows
      const int t = p >> 4, ch = p & 15;
      if constexpr (!PIPE) {
        const size_t o = vofs + (size_t)t * rsv + 8 * ch;
        store_tr_chunk<16>(sdR, t, ch, *reinterpret_cast<const u32x4*>(rw.src(dR + o, t)));
        store_tr_chunk<16>(sR, t, ch, *reinterpret_cast<const u32x4*>(rw.src(vnew + o, t)));
        store_tr_chunk<16>(sdO, t, ch, *reinterpret_cast<const u32x4*>(rw.src(dO + o, t)));
      }
    }
    int fb = 0;
    if (tid < C) {
      if constexpr (!VEC_B) {
        sBeta[tid] = pin.beta;
        fb = fabsf(pin.beta) < 1e-6f;
      }
      if constexpr (GATE == CG_SCALAR) sG[tid] = pin.g;
    }
    if (tid < KD) sGl[tid] = pin.gl;
    // block-uniform: some row has |beta| < 1e-6 (one flag per wave, then a barrier)
    const unsigned long long fbw = __ballot(fb);
    if (l == 0) sAny[wv] = fbw != 0ull;
    lds_sync();
#pragma unroll
    for (int w = 0; w < 8; ++w) any_fb |= sAny[w];
    if constexpr (ORIG) {
      // Z = beta v, E = beta k 2^g rows (bf16, swizzled) for T = dR Z^T + W-bar E^T
      bf16* sZ = reinterpret_cast<bf16*>(regA + LY::OFF_O);
      bf16* sE = sZ + C * KD;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int p = tid + 512 * i;
        const int t = p >> 4, ch = p & 15;
        const bf16x8 vv = *reinterpret_cast<const bf16x8*>(vb + (size_t)t * rsv + 8 * ch);
        const bf16x8 kx = *reinterpret_cast<const bf16x8*>(k + kofs + (size_t)t * rsk + 8 * ch);
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)t * rsk + 8 * ch);
        const f32x4 g1 = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)t * rsk + 8 * ch + 4);
        const float be = sBeta[t];
        bf16x8 z8, e8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          z8[j] = to_bf16(be * to_f32(vv[j]));
          e8[j] = to_bf16(be * to_f32(kx[j]) * fast_exp2(j < 4 ? g0[j] : g1[j - 4]));
        }
        store_tr_chunk<16>(sZ, t, ch, __builtin_bit_cast(u32x4, z8));
        store_tr_chunk<16>(sE, t, ch, __builtin_bit_cast(u32x4, e8));
      }
    }
    // persistent kernel: this item's q, k, g stream into region B during phases
    // 1-3 (issued after this phase's LDS writes, see dma_x's call below)
    if constexpr (PIPE) dma_qkg<GATE>(sQ, sK, sGr, q, k, g, pos, H, HQ, tid);
  }
  // the standalone intra adds the direct dbeta terms of every row
  const bool has_fb = !VEC_B && (INTRA || ORIG || any_fb != 0);
  f32x4 aq[4], ak[4], aw[4];                   // dq, dk, dG of column kk, rows 16 I + 4 lg + r
  float dgk = 0.f;

  if constexpr (!INTRA) {

  // ---------------- phase 1: P^T = dR^T A  (accumulator layout stores P row-major) ----------------
  {
    // LDS writes of P wait until every wave has read dR (P takes its place when
    // pipelined); sum_v P R goes to one LDS partial per column strip.  Each wave
    // takes one token tile from each half (t tiles th and 2 + th): the second half
    // needs half the contraction (A^T is upper triangular), so the waves balance.
    f32x4 pacc[2][2];
    float pra[2] = {0.f, 0.f};
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      const int vrow0 = 32 * cs + 16 * vt;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tcol0 = 16 * th + 32 * tt;
        f32x4& acc = pacc[vt][tt];
        acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks == 0 && tt == 1) continue;    // A^T upper triangular: s < 32 <= t vanishes
          const bf16x8 a = frag_tr<16>(sdR, 32 * ks, vrow0, l);          // dR^T rows v, over s
          acc = mfma(a, frag_tr<8>(sAh, 32 * ks, tcol0, l), acc);      // A[s][t] columns t, over s
          acc = mfma(a, frag_tr<8>(sAl, 32 * ks, tcol0, l), acc);
        }
        // lane: t = tcol0 + lc, v = vrow0 + 4 lg .. +3
        const int t = tcol0 + lc;
        const int v0 = vrow0 + 4 * lg;
        const size_t go = (size_t)t * rsv + v0;
        if constexpr (VEC_B) {
          const bf16x4 w4 = *reinterpret_cast<const bf16x4*>(rw.src(wgate + vofs + go, t));
          const bf16x4 x4 = *reinterpret_cast<const bf16x4*>(rw.src(vb + go, t));
          bf16x4 o1, o2;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            o1[r] = to_bf16(to_f32(w4[r]) * acc[r]);
            o2[r] = to_bf16(to_f32(x4[r]) * acc[r]);
          }
          *reinterpret_cast<bf16x4*>(rw.dst(dv_out + vofs + go, t)) = o1;
          *reinterpret_cast<bf16x4*>(rw.dst(dw_out + vofs + go, t)) = o2;
        } else {
          const float be = sBeta[t];
          const bf16x4 r4 = *reinterpret_cast<const bf16x4*>(sR + tr_off<16>(t, v0));
          bf16x4 o1;
          float pr = 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            o1[r] = to_bf16(be * acc[r]);
            pr += acc[r] * to_f32(r4[r]);
          }
          *reinterpret_cast<bf16x4*>(rw.dst(dv_out + vofs + go, t)) = o1;
          pra[tt] += sum_lane_groups(pr, l);
          if (has_fb) {
            const bf16x4 x4 = *reinterpret_cast<const bf16x4*>(rw.src(vb + go, t));
            float pv = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) pv += acc[r] * to_f32(x4[r]);
            pv = sum_lane_groups(pv, l);
            if (lg == 0) sFb[64 * (2 * cs + vt) + t] = pv;
          }
        }
      }
    }
    if constexpr (!VEC_B) {
      if (lg == 0) {
        sDbA[64 * cs + 16 * th + lc] = pra[0];
        sDbA[64 * cs + 32 + 16 * th + lc] = pra[1];
      }
    }
    if constexpr (PIPE) lds_sync();       // dR read by every wave: P overwrites it
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        bf16x4 p4;
#pragma unroll
        for (int r = 0; r < 4; ++r) p4[r] = to_bf16(pacc[vt][tt][r]);
        *reinterpret_cast<bf16x4*>(sP + tr_off<16>(16 * th + 32 * tt + lc, 32 * cs + 16 * vt + 4 * lg)) = p4;
      }
  }
  lds_sync();

  if constexpr (!PIPE) load_state();

  if constexpr (ORIG) {
    // ---------------- original formulation: W-bar, E-bar, T, J (D follows in phase 2) ----------------
    bf16* sZ = reinterpret_cast<bf16*>(regA + LY::OFF_O);
    bf16* sE = sZ + C * KD;
    bf16* sWb = sZ + 2 * C * KD;
    bf16* sTh = sZ;                   // T hi/lo [64][64] over Z (after T is formed)
    bf16* sTl = sZ + C * C;
    bf16* sJh = sE;                   // J hi/lo [64][64] over E
    bf16* sJl = sE + C * C;
    // W-bar strip = -dR h^T (this wave's 16 key columns, all 64 rows)
    f32x4 wb[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 z = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) z = mfma(frag_row<16>(sdR, 16 * I, 32 * ks, l), fh[ks], z);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        wb[I][r] = -z[r];
        sWb[tr_off<16>(16 * I + 4 * lg + r, kk)] = to_bf16(-z[r]);
      }
    }
    // E-bar strip = A^T W-bar (rows s, over t >= s), K = 16 MFMAs: the accumulator layout of
    // W-bar is the B layout; A^T's A operand is a transposed read of A's [t][s] rows.  The
    // residual code carries aw = P h^T = -E-bar, so aw = -E-bar here.
    auto mfma16 = [](bf16x4 a, bf16x4 b, f32x4 c) -> f32x4 {
      typedef short s4 __attribute__((ext_vector_type(4)));
      return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
    };
    bf16x4 wh[4], wl[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) wh[J] = split_hi4(wb[J], wl[J]);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 e = zero4();
#pragma unroll
      for (int J = I; J < 4; ++J) {
        const int o = tr_off<8>(16 * J + 4 * lg + (lc >> 2), 16 * I + 4 * (lc & 3));
        const bf16x4 ah = ds_read_tr4(sAh + o), al = ds_read_tr4(sAl + o);
        e = mfma16(ah, wh[J], e);
        e = mfma16(ah, wl[J], e);
        e = mfma16(al, wh[J], e);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) aw[I][r] = -e[r];
    }
    lds_sync();                       // W-bar complete
    // T = dR Z^T + W-bar E^T: wave (I = wv / 2) takes tiles (I, J) for J = 2 (wv & 1) + jj
    const int I = wv >> 1;
    f32x4 tt[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
      f32x4 a = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        a = mfma(frag_row<16>(sdR, 16 * I, 32 * ks, l), frag_row<16>(sZ, 16 * J, 32 * ks, l), a);
        a = mfma(frag_row<16>(sWb, 16 * I, 32 * ks, l), frag_row<16>(sE, 16 * J, 32 * ks, l), a);
      }
      tt[jj] = a;
    }
    lds_sync();                       // Z, E read: T hi/lo over Z
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bf16 hh, ll;
        split_bf16(tt[jj][r], hh, ll);
        const int o = tr_off<8>(16 * I + 4 * lg + r, 16 * J + lc);
        sTh[o] = hh;
        sTl[o] = ll;
      }
    }
    lds_sync();
    // J = A^T T (rows s, over t >= s)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int Jc = 2 * (wv & 1) + jj;
      f32x4 a = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (32 * ks + 31 < 16 * I) continue;      // A[t][s] = 0 for t < s
        const bf16x8 ah = frag_tr<8>(sAh, 32 * ks, 16 * I, l), al = frag_tr<8>(sAl, 32 * ks, 16 * I, l);
        const bf16x8 th = frag_tr<8>(sTh, 32 * ks, 16 * Jc, l), tl = frag_tr<8>(sTl, 32 * ks, 16 * Jc, l);
        a = mfma(ah, th, a);
        a = mfma(ah, tl, a);
        a = mfma(al, th, a);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bf16 hh, ll;
        split_bf16(a[r], hh, ll);
        const int o = tr_off<8>(16 * I + 4 * lg + r, 16 * Jc + lc);
        sJh[o] = hh;
        sJl[o] = ll;
      }
    }
    lds_sync();                       // J complete
  }

  // ---------------- phase 2: L = scale tril(dO R^T), D = -strict_tril(P R^T), both orientations ----------------
  if constexpr (ORIG) {
    // L as in the residual code; D^T tiles from J A^T (rows s, columns i): A's rows s read
    // along t, J's rows i along t.  Every wave reads A (region A) before any writes L / D
    // there, hence the barrier between the products and the stores.
    bf16* sJh = reinterpret_cast<bf16*>(regA + LY::OFF_O) + C * KD;
    bf16* sJl = sJh + C * C;
    const int I = wv >> 1;
    f32x4 bLs[2], bDs[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
      f32x4 bL = zero4(), bD = zero4();
      if (J >= I) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          bL = mfma(frag_row<16>(sR, 16 * I, 32 * ks, l), frag_row<16>(sdO, 16 * J, 32 * ks, l), bL);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const bf16x8 ah = frag_row<8>(sAh, 16 * I, 32 * ks, l), al = frag_row<8>(sAl, 16 * I, 32 * ks, l);
          const bf16x8 jh = frag_row<8>(sJh, 16 * J, 32 * ks, l), jl = frag_row<8>(sJl, 16 * J, 32 * ks, l);
          bD = mfma(ah, jh, bD);
          bD = mfma(ah, jl, bD);
          bD = mfma(al, jh, bD);
        }
      }
      bLs[jj] = bL;
      bDs[jj] = bD;
    }
    lds_sync();
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
      const int i = 16 * J + lc;
      f32x4 lv, dv4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s_ = 16 * I + 4 * lg + r;
        lv[r] = (i >= s_) ? scale * bLs[jj][r] : 0.f;
        dv4[r] = (i > s_) ? -bDs[jj][r] : 0.f;
      }
      bf16x4 lo;
      bf16x4 hi = split_hi4(lv, lo);
      *reinterpret_cast<bf16x4*>(Lrh + i * LDT + 16 * I + 4 * lg) = hi;
      *reinterpret_cast<bf16x4*>(Lrl + i * LDT + 16 * I + 4 * lg) = lo;
      hi = split_hi4(dv4, lo);
      *reinterpret_cast<bf16x4*>(Drh + i * LDT + 16 * I + 4 * lg) = hi;
      *reinterpret_cast<bf16x4*>(Drl + i * LDT + 16 * I + 4 * lg) = lo;
    }
  } else {
    const int I = wv >> 1;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
      // (a) tiles of L and D with rows i in block I, columns s in block J.  Their
      //     accumulator layout stores contiguously as L^T[s][i], D^T[s][i], the
      //     A operands of uk.
      // (b) tiles of L^T and D^T with rows s in block I, columns i in block J:
      //     they store contiguously as the row-major L[i][s], D[i][s].
      f32x4 aL = zero4(), aD = zero4(), bL = zero4(), bD = zero4();
      const bool lowerA = J <= I;      // (a) nonzero: s-block J <= i-block I
      const bool lowerB = J >= I;      // (b) nonzero: i-block J >= s-block I
      if (lowerA && LY::LT_COPY) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 br = frag_row<16>(sR, 16 * J, 32 * ks, l);
          aL = mfma(frag_row<16>(sdO, 16 * I, 32 * ks, l), br, aL);
          aD = mfma(frag_row<16>(sP, 16 * I, 32 * ks, l), br, aD);
        }
      }
      if (lowerB) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 ar = frag_row<16>(sR, 16 * I, 32 * ks, l);
          bL = mfma(ar, frag_row<16>(sdO, 16 * J, 32 * ks, l), bL);
          bD = mfma(ar, frag_row<16>(sP, 16 * J, 32 * ks, l), bD);
        }
      }
      if constexpr (LY::LT_COPY) {
        // (a): lane holds rows i = 16 I + 4 lg + r, column s = 16 J + lc
        const int s = 16 * J + lc;
        f32x4 lv, dv4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lg + r;
          float f = 1.f;
          if constexpr (GATE == CG_SCALAR) f = (i >= s) ? fast_exp2(sG[i] - sG[s]) : 0.f;
          lv[r] = (i >= s) ? scale * aL[r] * f : 0.f;
          dv4[r] = (i > s) ? -aD[r] * f : 0.f;
        }
        bf16x4 lo;
        bf16x4 hi = split_hi4(lv, lo);
        *reinterpret_cast<bf16x4*>(Lth + s * LDT + 16 * I + 4 * lg) = hi;
        *reinterpret_cast<bf16x4*>(Ltl + s * LDT + 16 * I + 4 * lg) = lo;
        hi = split_hi4(dv4, lo);
        *reinterpret_cast<bf16x4*>(Dth + s * LDT + 16 * I + 4 * lg) = hi;
        *reinterpret_cast<bf16x4*>(Dtl + s * LDT + 16 * I + 4 * lg) = lo;
      }
      {
        // (b): lane holds rows s = 16 I + 4 lg + r, column i = 16 J + lc
        const int i = 16 * J + lc;
        f32x4 lv, dv4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 16 * I + 4 * lg + r;
          float f = 1.f;
          if constexpr (GATE == CG_SCALAR) f = (i >= s) ? fast_exp2(sG[i] - sG[s]) : 0.f;
          lv[r] = (i >= s) ? scale * bL[r] * f : 0.f;
          dv4[r] = (i > s) ? -bD[r] * f : 0.f;
        }
        bf16x4 lo;
        bf16x4 hi = split_hi4(lv, lo);
        *reinterpret_cast<bf16x4*>(Lrh + i * LDT + 16 * I + 4 * lg) = hi;
        *reinterpret_cast<bf16x4*>(Lrl + i * LDT + 16 * I + 4 * lg) = lo;
        hi = split_hi4(dv4, lo);
        *reinterpret_cast<bf16x4*>(Drh + i * LDT + 16 * I + 4 * lg) = hi;
        *reinterpret_cast<bf16x4*>(Drl + i * LDT + 16 * I + 4 * lg) = lo;
        // the WY seam's dA: row i, columns s = 16 I + 4 lg .. + 3 (zero on and above the diagonal)
        if constexpr (WY)
          *reinterpret_cast<f32x4*>(rw.dst(dA_wy + (tok0 * H + h) * C + (size_t)i * rsa + 16 * I + 4 * lg, i)) = dv4;
      }
    }
  }   // phase 2

  // ---------------- phase 3: dq_s = dO h^T, dk_s = R dh^T, dw = P h^T (16-column strip, 64 rows) ----------------
  {
    float sacc = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) sacc += to_f32(fh[ks][j]) * to_f32(fdh[ks][j]);
    dgk = sum_lane_groups(sacc, l);               // sum_v h[kk][v] dh[kk][v]
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 x = zero4(), y = zero4(), z = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        x = mfma(frag_row<16>(sdO, 16 * I, 32 * ks, l), fh[ks], x);
        y = mfma(frag_row<16>(sR, 16 * I, 32 * ks, l), fdh[ks], y);
        if constexpr (!ORIG) z = mfma(frag_row<16>(sP, 16 * I, 32 * ks, l), fh[ks], z);
      }
      aq[I] = x;
      ak[I] = y;
      if constexpr (!ORIG) aw[I] = z;
    }
  }
  }   // !INTRA: phases 1-3

  if constexpr (PIPE) {
    // q, k, g were copied into region B at the item start: each wave waits for
    // its own copies, the barrier publishes them (and retires P, R, dO)
    __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0)
    lds_sync();
    // The next item's dR, R, dO stream into X during phases 4-6 (the copies are
    // asm, outside the compiler's wait counts, so the branch costs no precision).
    if (next_item >= 0) dma_x(xbuf, dR, vnew, dO, ChunkItem(next_item, T, H), H, tid);
  } else {
    // q, k, g (and b) rows for the row-major staging (issued before the barrier)
    u32x4 rq[2], rk[2], rb[2];
    f32x4 rg[4];
    const QKRows qr = qk_rows(tok0, h, H, HQ);       // raw q / k (grouped value heads: HQ < H)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;
      const size_t o = kofs + (size_t)(p >> 4) * rsk + (p & 15) * 8;
      const size_t oq = qr.ofs + (size_t)(p >> 4) * qr.rs + (p & 15) * 8;
      rq[i] = *reinterpret_cast<const u32x4*>(rw.src(q + oq, p >> 4));
      rk[i] = *reinterpret_cast<const u32x4*>(rw.src(k + oq, p >> 4));
      if constexpr (VEC_B) rb[i] = *reinterpret_cast<const u32x4*>(rw.src(bgate + o, p >> 4));
    }
    if constexpr (GATE == CG_VECTOR) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = tid + 512 * i;              // 2048 pieces: token p >> 5, 4 columns
        rg[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rw.clamp(p >> 5) * rsk + (p & 31) * 4);
      }
    }
    lds_sync();   // P, R, dO no longer needed: region B becomes q, k, g (, b)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;
      store_tr_chunk<16>(sQ, p >> 4, p & 15, rq[i]);
      store_tr_chunk<16>(sK, p >> 4, p & 15, rk[i]);
      if constexpr (VEC_B) store_tr_chunk<16>(sB, p >> 4, p & 15, rb[i]);
    }
    if constexpr (GATE == CG_VECTOR) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = tid + 512 * i;
        *reinterpret_cast<f32x4*>(sGr + g_off(p >> 5, (p & 31) * 4)) = rg[i];
      }
    }
    lds_sync();
  }

  // ---------------- per-lane operands of column kk, rows 16 J + 4 lg + j ----------------
  // In the accumulator layout and in the B layout of the K=16 MFMA a lane holds the
  // same four rows of one column, so one set of per-element values serves the
  // epilogue, the intra operands and the output scaling.
  f32x4 g4[4];
  bf16x4 qb4[4], kb4[4];
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    const int r0 = 16 * J + 4 * lg;
    if constexpr (GATE == CG_VECTOR) {
#pragma unroll
      for (int j = 0; j < 4; ++j) g4[J][j] = sGr[g_off(r0 + j, kk)];
    }
    else if constexpr (GATE == CG_SCALAR) g4[J] = *reinterpret_cast<const f32x4*>(sG + r0);
    else g4[J] = zero4();
    // transposed reads: rows r0 .. r0 + 3 of column kk
    const int tro = tr_off<16>(r0 + (lc >> 2), 16 * wv + 4 * (lc & 3));
    qb4[J] = ds_read_tr4(sQ + tro);
    kb4[J] = ds_read_tr4(sK + tro);
  }
  // erase gate of rows 16 J + 4 lg .. +3 (reloaded from LDS where needed)
  auto bvals = [&](int J) -> f32x4 {
    const int r0 = 16 * J + 4 * lg;
    if constexpr (VEC_B) {
      const bf16x4 bq = ds_read_tr4(sB + tr_off<16>(r0 + (lc >> 2), 16 * wv + 4 * (lc & 3)));
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = to_f32(bq[j]);
      return o;
    } else {
      return *reinterpret_cast<const f32x4*>(sBeta + r0);
    }
  };
  // gate extremes of each 16-row block (this column) and the per-element ratios
  //   EB = 2^(bot_J - g) <= 1,  ET = 2^(g - top_J) <= 1
  float top[4], bot[4];
  bool pair[4];
  f32x4 EB[4], ET[4];
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    float hi = fmaxf(fmaxf(g4[J][0], g4[J][1]), fmaxf(g4[J][2], g4[J][3]));
    float lo = fminf(fminf(g4[J][0], g4[J][1]), fminf(g4[J][2], g4[J][3]));
    hi = fmaxf(hi, lane_xor16(hi));
    hi = fmaxf(hi, lane_read(hi, l ^ 32));
    lo = fminf(lo, lane_xor16(lo));
    lo = fminf(lo, lane_read(lo, l ^ 32));
    top[J] = hi;
    bot[J] = lo;
    pair[J] = (GATE == CG_VECTOR) && (hi - lo) >= 80.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      EB[J][j] = (GATE == CG_VECTOR) ? fast_exp2(lo - g4[J][j]) : 1.f;
      ET[J][j] = (GATE == CG_VECTOR) ? fast_exp2(g4[J][j] - hi) : 1.f;
    }
  }
  const float gl = sGl[kk];

  // ---------------- phase 4: state-gradient epilogue ----------------
  float colkdk = 0.f;
  f32x4 fbrow[4];      // scalar-beta fallback rows: k exp2(g) Eb + k ue, summed over columns later
  f32x4 adb[4];        // vector-b family: db = k exp2(g) Eb + k ue
  if constexpr (INTRA) {
    // the intra terms alone; the partial gradients are added at the stores (not held
    // in registers through phase 5)
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      aq[I] = zero4();
      ak[I] = zero4();
      aw[I] = zero4();
      if constexpr (VEC_B) adb[I] = zero4();
      else fbrow[I] = zero4();
    }
  } else {
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    float gtop = 1.f, gdec = 1.f;
    if constexpr (GATE == CG_VECTOR) {
      gtop = fast_exp2(top[I]);            // exp2(g_i) = exp2(top) * ET
      gdec = fast_exp2(gl - bot[I]);       // exp2(g_last - g_i) = exp2(g_last - bot) * EB
    }
    const f32x4 b4 = bvals(I);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float gam = 1.f, kdec = 1.f;
      if constexpr (GATE == CG_VECTOR) {
        gam = gtop * ET[I][r];
        kdec = gdec * EB[I][r];
      } else if constexpr (GATE == CG_SCALAR) {
        gam = fast_exp2(g4[I][r]);
        kdec = fast_exp2(gl - g4[I][r]);
      }
      const float qv = to_f32(qb4[I][r]), kv = to_f32(kb4[I][r]), bv = b4[r];
      const float dqv = aq[I][r] * gam * scale;
      const float dks = ak[I][r] * kdec;
      const float eb = -aw[I][r];
      const float keb = kv * gam * eb;
      aq[I][r] = dqv;
      ak[I][r] = dks + bv * gam * eb;
      aw[I][r] = qv * dqv - kv * dks + bv * keb;
      colkdk += kv * dks;
      if constexpr (VEC_B) adb[I][r] = keb;
      else fbrow[I][r] = keb;
    }
  }
  }   // !INTRA: phase 4

  // ---------------- phase 5: matrix intra ----------------
  if constexpr (!WY) {
  auto combine = [&](int I, const f32x4& xq, const f32x4& xe, const f32x4& xk) {
    const f32x4 b4 = bvals(I);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float qv = to_f32(qb4[I][r]), kv = to_f32(kb4[I][r]), bv = b4[r];
      aq[I][r] += xq[r];
      ak[I][r] += bv * xe[r] + xk[r];
      aw[I][r] += qv * xq[r] + kv * (bv * xe[r] - xk[r]);
      if constexpr (VEC_B) adb[I][r] += kv * xe[r];
      else fbrow[I][r] += xe[r] * kv;
    }
  };
  if constexpr (GATE != CG_VECTOR) {
    // Scalar / no gate: L and D already carry the gate (phase 2), so the intra
    // products are plain triangular matmuls, K = 32 MFMAs with every operand read
    // straight from LDS: uq = L k, ue = D k (rows i, s <= i), uk = L^T q + D^T (beta k)
    // (s >= i); L^T and D^T come from transposed reads, k and q are exact bf16.
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 xq = zero4(), xe = zero4(), xk = zero4();
#pragma unroll
      for (int ks = 0; ks <= (16 * I + 15) / 32; ++ks) {
        const bf16x8 bk = frag_tr<16>(sK, 32 * ks, 16 * wv, l);
        xq = mfma(frag(Lrh + (16 * I) * LDT + 32 * ks, LDT, l), bk, xq);
        xq = mfma(frag(Lrl + (16 * I) * LDT + 32 * ks, LDT, l), bk, xq);
        xe = mfma(frag(Drh + (16 * I) * LDT + 32 * ks, LDT, l), bk, xe);
        xe = mfma(frag(Drl + (16 * I) * LDT + 32 * ks, LDT, l), bk, xe);
      }
#pragma unroll
      for (int ks = (16 * I) / 32; ks < 2; ++ks) {
        const bf16x8 bq = frag_tr<16>(sQ, 32 * ks, 16 * wv, l);
        const bf16x8 bk = frag_tr<16>(sK, 32 * ks, 16 * wv, l);
        bf16x8 bkh, bkl;                          // beta_s k_s, rows s = 32 ks + 8 lg + j
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          bf16 hh, ll;
          split_bf16(sBeta[32 * ks + 8 * lg + j] * to_f32(bk[j]), hh, ll);
          bkh[j] = hh;
          bkl[j] = ll;
        }
        const bf16x8 lth = frag_tr_pitch(Lrh, LDT, 32 * ks, 16 * I, l);
        const bf16x8 ltl = frag_tr_pitch(Lrl, LDT, 32 * ks, 16 * I, l);
        const bf16x8 dth = frag_tr_pitch(Drh, LDT, 32 * ks, 16 * I, l);
        const bf16x8 dtl = frag_tr_pitch(Drl, LDT, 32 * ks, 16 * I, l);
        xk = mfma(lth, bq, xk);
        xk = mfma(ltl, bq, xk);
        xk = mfma(dth, bkh, xk);
        xk = mfma(dth, bkl, xk);
        xk = mfma(dtl, bkh, xk);
      }
      combine(I, xq, xe, xk);
    }
  } else {
  // vector gates: K=16 MFMAs per 16-row sub-block
  // B operands (shared by every output block): kE = k EB, qE = q ET, bkE = b k ET,
  // split into bf16 hi + lo.  Sub-block J contributes to output block I with the
  // per-column factor 2^(top_I - bot_J) (uq, ue; J <= I) or 2^(top_J - bot_I) (uk; J >= I),
  // and the per-row factor ET_i (uq, ue) or EB_i (uk).
  bf16x4 kEh[4], kEl[4], qEh[4], qEl[4], eEh[4], eEl[4];
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    const f32x4 b4 = bvals(J);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float kv = to_f32(kb4[J][j]);
      bf16 h_, l_;
      split_bf16(kv * EB[J][j], h_, l_);
      kEh[J][j] = h_;
      kEl[J][j] = l_;
      split_bf16(to_f32(qb4[J][j]) * ET[J][j], h_, l_);
      qEh[J][j] = h_;
      qEl[J][j] = l_;
      split_bf16(b4[j] * kv * ET[J][j], h_, l_);
      eEh[J][j] = h_;
      eEl[J][j] = l_;
    }
  }
  auto mfma16 = [](bf16x4 a, bf16x4 b, f32x4 c) -> f32x4 {
    typedef short s4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
  };
  auto afrag4 = [&](const bf16* base) -> bf16x4 {   // rows (lc), cols 4 lg .. 4 lg + 3
    return *reinterpret_cast<const bf16x4*>(base + lc * LDT + 4 * lg);
  };
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    f32x4 xq = zero4(), xe = zero4(), xk = zero4();
#pragma unroll
    for (int J = 0; J <= I; ++J) {
      // MFMA operands are read from all 64 lanes, so fragments are loaded and the
      // products issued for every lane; a pairwise column (diagonal block with a
      // wide gate span) drops its own result through a zero factor instead.
      const bf16x4 lh = afrag4(Lrh + (16 * I) * LDT + 16 * J), ll = afrag4(Lrl + (16 * I) * LDT + 16 * J);
      const bf16x4 dh_ = afrag4(Drh + (16 * I) * LDT + 16 * J), dl_ = afrag4(Drl + (16 * I) * LDT + 16 * J);
      f32x4 a = zero4(), e = zero4();
      a = mfma16(lh, kEh[J], a);
      a = mfma16(lh, kEl[J], a);
      a = mfma16(ll, kEh[J], a);
      e = mfma16(dh_, kEh[J], e);
      e = mfma16(dh_, kEl[J], e);
      e = mfma16(dl_, kEh[J], e);
      float cf = (GATE == CG_VECTOR) ? fast_exp2(top[I] - bot[J]) : 1.f;
      if (J == I && pair[I]) cf = 0.f;        // exact pairwise diagonal below
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xq[r] += cf * a[r];
        xe[r] += cf * e[r];
      }
    }
#pragma unroll
    for (int J = I; J < 4; ++J) {
      bf16x4 lh, ll, dh_, dl_;
      if constexpr (LY::LT_COPY) {
        lh = afrag4(Lth + (16 * I) * LDT + 16 * J);
        ll = afrag4(Ltl + (16 * I) * LDT + 16 * J);
        dh_ = afrag4(Dth + (16 * I) * LDT + 16 * J);
        dl_ = afrag4(Dtl + (16 * I) * LDT + 16 * J);
      } else {
        // transposed reads of the row-major tiles: lane gets L[16 J + 4 lg + j][16 I + lc]
        const int o = (16 * J + 4 * lg + (lc >> 2)) * LDT + 16 * I + 4 * (lc & 3);
        lh = ds_read_tr4(Lrh + o);
        ll = ds_read_tr4(Lrl + o);
        dh_ = ds_read_tr4(Drh + o);
        dl_ = ds_read_tr4(Drl + o);
      }
      f32x4 a = zero4();
      a = mfma16(lh, qEh[J], a);
      a = mfma16(lh, qEl[J], a);
      a = mfma16(ll, qEh[J], a);
      a = mfma16(dh_, eEh[J], a);
      a = mfma16(dh_, eEl[J], a);
      a = mfma16(dl_, eEh[J], a);
      float cf = (GATE == CG_VECTOR) ? fast_exp2(top[J] - bot[I]) : 1.f;
      if (J == I && pair[I]) cf = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) xk[r] += cf * a[r];
    }
    if constexpr (GATE == CG_VECTOR) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xq[r] *= ET[I][r];
        xe[r] *= ET[I][r];
        xk[r] *= EB[I][r];
      }
      if (pair[I]) {   // exact pairwise diagonal block (gate span >= 80 in log2 units)
#pragma unroll 1
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lg + r;
          const float gi = sGr[g_off(i, kk)];
          float pq = 0.f, pe = 0.f, pk = 0.f;
#pragma unroll 1
          for (int s = 16 * I; s < 16 * (I + 1); ++s) {
            const float gs = sGr[g_off(s, kk)];
            const float ksv = to_f32(sK[tr_off<16>(s, kk)]);
            if (s <= i) {
              const float f = fast_exp2(gi - gs);
              pq += (to_f32(Lrh[i * LDT + s]) + to_f32(Lrl[i * LDT + s])) * ksv * f;
              if (s < i) pe += (to_f32(Drh[i * LDT + s]) + to_f32(Drl[i * LDT + s])) * ksv * f;
            }
            if (s >= i) {
              const float f = fast_exp2(gs - gi);
              const float lsi = to_f32(Lrh[s * LDT + i]) + to_f32(Lrl[s * LDT + i]);
              const float dsi = to_f32(Drh[s * LDT + i]) + to_f32(Drl[s * LDT + i]);
              float bs;
              if constexpr (VEC_B) bs = to_f32(sB[tr_off<16>(s, kk)]);
              else bs = sBeta[s];
              pk += (lsi * to_f32(sQ[tr_off<16>(s, kk)]) + dsi * bs * ksv) * f;
            }
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            if (rr == r) {
              xq[rr] += pq;
              xe[rr] += pe;
              xk[rr] += pk;
            }
          }
        }
      }
    }
    combine(I, xq, xe, xk);
  }

  }   // vector gates
  }   // !WY: phase 5

  // fallback dbeta rows: direct terms sum_k (k exp2(g) Eb + k ue), summed over all columns
  if constexpr (!VEC_B) {
    if (has_fb) {
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float s = sum_row16(fbrow[I][r]);
          if (lc == 0) sFb[512 + 64 * wv + 16 * I + 4 * lg + r] = s;
        }
    }
  }

  // ---------------- phase 6: last-row state terms, reverse cumsum, stores ----------------
  if constexpr (!INTRA) {
  colkdk = sum_lane_groups(colkdk, l);            // sum over the 64 rows of k dks (this column)
  if constexpr (GATE == CG_VECTOR) {
    const float term = fast_exp2(gl) * dgk + colkdk;
    if (lg == 3) aw[3][3] += term;
    float carry = 0.f;                         // total of the rows below
#pragma unroll
    for (int I = 3; I >= 0; --I) {
      if constexpr (WY) break;                 // the seam's dg stays before the cumsum
      f32x4& x = aw[I];
      x[2] += x[3];
      x[1] += x[2];
      x[0] += x[1];
      const float tot = x[0];                  // this lane group's 4-row total
      const float t0 = lane_read(tot, lc);
      const float t1 = lane_read(tot, lc + 16);
      const float t2 = lane_read(tot, lc + 32);
      const float t3 = lane_read(tot, lc + 48);
      float below = carry;
      if (lg < 3) below += t3;
      if (lg < 2) below += t2;
      if (lg < 1) below += t1;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] += below;
      carry += t0 + t1 + t2 + t3;
    }
  } else if constexpr (GATE == CG_SCALAR) {
    // scalar gate: dG row sums over this wave's 16 columns (one partial per wave),
    // the last row adding the state term
    const float term = sum_row16(fast_exp2(gl) * dgk + colkdk);
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s = sum_row16(aw[I][r]);
        if (I == 3 && r == 3 && lg == 3) s += term;
        if (lc == 0) sDg[64 * wv + 16 * I + 4 * lg + r] = s;
      }
  }
  }   // !INTRA: phase 6

  if constexpr (PIPE) {
    // the next item's prefetch (issued after phase 3) has landed in this wave's
    // rows; its A goes to registers before this item's stores are issued
    __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0)
    load_phase_in<GATE, VEC_B>(akk, beta, g, ChunkItem(next_item >= 0 ? next_item : item, T, H), H, tid, pin);
    asm volatile("" ::: "memory");          // the loads stay ahead of the stores below
  }
  // stores of dq, dk (bf16), the vector dg (fp32) and db (bf16); 32-bit offsets
  // from uniform per-chunk-head bases
  if constexpr (INTRA) {
    const int rsk32 = H * KD;
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * I + 4 * lg + r;
        const int off = t * rsk32 + kk;
        if (!rw.ok(t)) continue;            // a packed batch's missing rows
        dq32[kofs + off] += aq[I][r];
        dk32[kofs + off] += ak[I][r];
        dg_out[kofs + off] += aw[I][r];
        if constexpr (VEC_B) db32[kofs + off] += adb[I][r];
      }
  } else {
    bf16* dqb = dq_out + kofs;
    bf16* dkb = dk_out + kofs;
    float* dgb = dg_out + kofs;
    bf16* dbb = db_out + kofs;
    const int rsk32 = H * KD;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * I + 4 * lg + r;
        const int off = t * rsk32 + kk;
        if constexpr (WY) {
          *rw.dst(dq32 + kofs + off, t) = aq[I][r];
          *rw.dst(dk32 + kofs + off, t) = ak[I][r];
        } else {
          *rw.dst(dqb + off, t) = to_bf16(aq[I][r]);
          *rw.dst(dkb + off, t) = to_bf16(ak[I][r]);
        }
        if constexpr (GATE == CG_VECTOR && FOLD < 0) *rw.dst(dgb + off, t) = aw[I][r];
        if constexpr (VEC_B) {
          if constexpr (WY) *rw.dst(db32 + kofs + off, t) = adb[I][r];   // the intra adds ue k
          else *rw.dst(dbb + off, t) = to_bf16(adb[I][r]);
        }
      }
    }
    if constexpr (FOLD >= 0) {
      // dx = dg * d(activation)/dx at each row of this lane's column; the column's
      // sum over the 64 rows (ddt_bias) and the dA_log terms go to per-chunk partials
      constexpr int MODE = FOLD >> 1;
      constexpr bool RB = FOLD & 1;
      const int hh = pos.h, col = hh * KD + kk;
      const size_t base = kofs + (size_t)(4 * lg) * rsk32 + kk;
      float xr[4][4];
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t o = base + (size_t)(16 * I + r) * rsk32;
          const int t = 16 * I + 4 * lg + r;
          if constexpr (RB) xr[I][r] = to_f32(*rw.src(reinterpret_cast<const bf16*>(gf->graw) + o, t));
          else xr[I][r] = *rw.src(reinterpret_cast<const float*>(gf->graw) + o, t);
        }
      const float bias = gf->dt_bias ? gf->dt_bias[col] : 0.f;
      const float a = MODE == 2 ? 1.f : exp_f(gf->A_log[hh]);
      const float lb = gf->lower_bound;
      float sdt = 0.f, sda = 0.f;
#pragma unroll
      for (int I = 0; I < 4; ++I) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t o = base + (size_t)(16 * I + r) * rsk32;
          const float x = xr[I][r] + bias, d = aw[I][r];
          float dx, tda;
          if constexpr (MODE == 0) {
            const float y = exp_f(x);
            dx = -d * a * sigmoid_y(y);
            tda = d * (-a * softplus_y(x, y));
          } else {
            const float sg = sigmoid_y(exp_f(a * x));
            const float ds = d * lb * sg * (1.f - sg);
            dx = ds * a;
            tda = MODE == 1 ? ds * a * x : 0.f;
          }
          if constexpr (RB) *rw.dst(reinterpret_cast<bf16*>(gf->dx) + o, 16 * I + 4 * lg + r) = to_bf16(dx);
          else *rw.dst(reinterpret_cast<float*>(gf->dx) + o, 16 * I + 4 * lg + r) = dx;
          if (!rw.ok(16 * I + 4 * lg + r)) dx = tda = 0.f;   // rows past a sequence's end
          sdt += dx;
          sda += tda;
        }
      }
      sdt = sum_lane_groups(sdt, l);             // the column's 64 rows
      sda = sum_row16(sum_lane_groups(sda, l));  // and the strip's 16 columns
      const int NT = T / C;
      const size_t blk = (size_t)pos.b * NT + pos.c;
      if (lg == 0) gf->part_dt[blk * (H * KD) + col] = sdt;
      if (l == 0) gf->part_da[(blk * H + hh) * 8 + wv] = sda;
    }
  }
  lds_sync();   // sFb, sDg complete; every wave is past phase 5 (region A free)
  if constexpr (PIPE) {
    // The next item's A: wait for its loads (issued ahead of this item's stores,
    // one store per row and output below) without waiting for the stores, and
    // stage it into region A.
    constexpr int STORES = 16 * (2 + (GATE == CG_VECTOR ? 1 : 0) + (VEC_B ? 1 : 0));
    static_assert(STORES < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(STORES));
    stage_akk(pin, sAh, sAl, tid);
  }
  // the fallback rows' direct dbeta: phase-1 partials (one per column strip and value tile),
  // then phase 5's (one per wave), in a fixed order; only where written (has_fb, uniform)
  float fbs = 0.f;
  if constexpr (!VEC_B) {
    if (has_fb && tid < C) {
      if constexpr (!INTRA) {
#pragma unroll
        for (int j = 0; j < 8; ++j) fbs += sFb[64 * j + tid];
      }
#pragma unroll
      for (int w = 0; w < 8; ++w) fbs += sFb[512 + 64 * w + tid];
    }
  }
  if (INTRA && tid < C) {
    // endpoint_intra.py:190-194: every row, or only |beta| < 1e-6 rows when the
    // residual producer already accounted for the rest (beta_complete)
    if constexpr (!VEC_B) {
      const size_t row = (tok0 + tid) * H + h;
      if (rw.ok(tid) && (!beta_complete || fabsf(sBeta[tid]) < 1e-6f)) dbeta_out[row] += fbs;
    }
  } else if (tid < C) {
    const size_t row = (tok0 + tid) * H + h;
    if constexpr (!VEC_B) {
      const float be = sBeta[tid];
      const float pr = (sDbA[tid] + sDbA[64 + tid]) + (sDbA[128 + tid] + sDbA[192 + tid]);
      float db = (ORIG || fabsf(be) < 1e-6f) ? fbs : pr / be;
      // beta = s sigmoid(x) activated in the forward (use_beta_sigmoid_in_kernel):
      // dL/dx = dL/dbeta * s sigmoid (1 - sigmoid) = dL/dbeta * beta (1 - beta / s)
      if (beta_sig > 0.f) db *= be * (1.f - be / beta_sig);
      *rw.dst(dbeta_out + row, tid) = db;
    }
    if constexpr (GATE == CG_SCALAR) {
      // row sums over the 8 waves' partials, then the reverse cumsum over the
      // 64 rows as a suffix scan across the lanes of wave 0
      float x = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) x += sDg[64 * w + tid];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = lane_read(x, l + d < 64 ? l + d : 63);
        if (l + d < 64) x += y;
      }
      *rw.dst(dg_out + row, tid) = x;
    }
  }
  // persistent kernel: every wave's prefetch complete and this item's LDS reads
  // done before the next item's phase 0
  if constexpr (PIPE) lds_sync();
}

template <int GATE, bool VEC_B, bool HVF = false, bool MAP = false>
__global__ __launch_bounds__(512) void chunk_bwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const bf16* __restrict__ hst,
    const bf16* __restrict__ dhst, bf16* __restrict__ dq_out, bf16* __restrict__ dk_out,
    bf16* __restrict__ dv_out, float* __restrict__ dg_out, float* __restrict__ dbeta_out,
    bf16* __restrict__ db_out, bf16* __restrict__ dw_out, int T, int H, float scale, float beta_sig, int HQ,
    const int* __restrict__ cu, const int* __restrict__ ci) {
  using LY = PostLayout<GATE, VEC_B>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PhaseIn pin;
  chunk_body<GATE, VEC_B, false, false, -1, HVF, false, MAP>(
      q, k, v, vnew, dO, dR, g, beta, bgate, wgate, akk, hst, dhst, dq_out, dk_out, dv_out, dg_out, dbeta_out, db_out,
      dw_out, T, H, scale, nullptr, nullptr, nullptr, nullptr, 0, blockIdx.x, -1, smem, smem + LY::REGION_A,
      reinterpret_cast<float*>(smem + LY::REGION_A + LY::REGION_B), nullptr, nullptr, pin, nullptr, beta_sig, HQ, cu,
      ci);
}

// KDA in the original 7-product formulation (the same-GPU comparator, ORIG above)
template <int DUMMY = 0>
__global__ __launch_bounds__(512) void chunk_bwd_original_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const float* __restrict__ akk,
    const bf16* __restrict__ hst, const bf16* __restrict__ dhst, bf16* __restrict__ dq_out,
    bf16* __restrict__ dk_out, bf16* __restrict__ dv_out, float* __restrict__ dg_out,
    float* __restrict__ dbeta_out, int T, int H, float scale) {
  using LY = PostLayout<CG_VECTOR, false, false, false, true>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PhaseIn pin;
  chunk_body<CG_VECTOR, false, false, false, -1, false, true>(
      q, k, v, vnew, dO, dR, g, beta, nullptr, nullptr, akk, hst, dhst, dq_out, dk_out, dv_out, dg_out, dbeta_out,
      nullptr, nullptr, T, H, scale, nullptr, nullptr, nullptr, nullptr, 0, blockIdx.x, -1, smem,
      smem + LY::REGION_A, reinterpret_cast<float*>(smem + LY::REGION_A + LY::REGION_B), nullptr, nullptr, pin);
}

// The kernel-level WY seams (every term but the matrix intra; see WY above): KDA (scalar
// beta) and GDN2 (VEC_B: erase gate b, write gate w; db in fp32 for the intra to complete,
// dw complete); MAP: a packed variable-length batch (cu, ci as for chunk_bwd_kernel)
template <bool VEC_B, bool HVF, bool MAP>
__global__ __launch_bounds__(512) void chunk_bwd_wy_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const bf16* __restrict__ hst,
    const bf16* __restrict__ dhst, float* __restrict__ dq32, float* __restrict__ dk32, bf16* __restrict__ dv_out,
    float* __restrict__ dg_out, float* __restrict__ dbeta_out, float* __restrict__ db32, bf16* __restrict__ dw_out,
    float* __restrict__ dA, int T, int H, float scale, int HQ, const int* __restrict__ cu,
    const int* __restrict__ ci) {
  using LY = PostLayout<CG_VECTOR, VEC_B>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PhaseIn pin;
  chunk_body<CG_VECTOR, VEC_B, false, false, -1, HVF, false, MAP, true>(
      q, k, v, vnew, dO, dR, g, beta, bgate, wgate, akk, hst, dhst, nullptr, nullptr, dv_out, dg_out, dbeta_out,
      nullptr, dw_out, T, H, scale, nullptr, dq32, dk32, db32, 0, blockIdx.x, -1, smem, smem + LY::REGION_A,
      reinterpret_cast<float*>(smem + LY::REGION_A + LY::REGION_B), nullptr, nullptr, pin, nullptr, 0.f, HQ, cu,
      ci, dA);
}

// KDA with the gate backward folded into the dg stores (no dg output); MAP: a packed
// variable-length batch (cu, ci as for chunk_bwd_kernel)
template <int FOLD, bool HVF = false, bool MAP = false>
__global__ __launch_bounds__(512) void chunk_bwd_fold_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const float* __restrict__ akk,
    const bf16* __restrict__ hst, const bf16* __restrict__ dhst, bf16* __restrict__ dq_out,
    bf16* __restrict__ dk_out, bf16* __restrict__ dv_out, float* __restrict__ dbeta_out, int T, int H,
    float scale, GateFoldArgs gf, float beta_sig, int HQ, const int* __restrict__ cu,
    const int* __restrict__ ci) {
  using LY = PostLayout<CG_VECTOR, false>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PhaseIn pin;
  chunk_body<CG_VECTOR, false, false, false, FOLD, HVF, false, MAP>(
      q, k, v, vnew, dO, dR, g, beta, nullptr, nullptr, akk, hst, dhst, dq_out, dk_out, dv_out, nullptr, dbeta_out,
      nullptr, nullptr, T, H, scale, nullptr, nullptr, nullptr, nullptr, 0, blockIdx.x, -1, smem,
      smem + LY::REGION_A, reinterpret_cast<float*>(smem + LY::REGION_A + LY::REGION_B), nullptr, nullptr, pin,
      &gf, beta_sig, HQ, cu, ci);
}

// Persistent form: one work-group per CU walks the items blockIdx.x, + gridDim.x, ...
// The next item's dR, R, dO are copied straight into LDS (and its A and per-row
// scalars into registers) while the current one computes phases 4-6, and an
// item's q, k, g while it computes phases 0-3, so that HBM reads overlap the
// matrix work instead of stalling the work-group.  Measured slower for KDA (its
// chunk kernel is bound by HBM bandwidth, not by exposed latency), so KDA keeps
// one work-group per chunk-head.
template <int GATE, bool VEC_B>
__global__ __launch_bounds__(512) void chunk_bwd_pipe_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const bf16* __restrict__ hst,
    const bf16* __restrict__ dhst, bf16* __restrict__ dq_out, bf16* __restrict__ dk_out,
    bf16* __restrict__ dv_out, float* __restrict__ dg_out, float* __restrict__ dbeta_out,
    bf16* __restrict__ db_out, bf16* __restrict__ dw_out, int T, int H, float scale, int items,
    float beta_sig, int HQ) {
  using LY = PostLayout<GATE, VEC_B, false, true>;
  __shared__ __attribute__((aligned(16))) bf16 xbuf[3 * C * KD];
  __shared__ __attribute__((aligned(16))) char regA[LY::REGION_A];
  __shared__ __attribute__((aligned(16))) char regB[LY::REGION_B];
  __shared__ __attribute__((aligned(16))) float small[LY::S_N];
  __shared__ __attribute__((aligned(16))) float gbuf[LY::GT_BYTES > 0 ? C * KD : 4];
  PhaseIn pin;
  int it = blockIdx.x;
  if (it >= items) return;
  {
    const ChunkItem first(it, T, H);
    dma_x(xbuf, dR, vnew, dO, first, H, threadIdx.x);
    load_phase_in<GATE, VEC_B>(akk, beta, g, first, H, threadIdx.x, pin);
    __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0)
    stage_akk(pin, reinterpret_cast<bf16*>(regA + LY::OFF_AKTH), reinterpret_cast<bf16*>(regA + LY::OFF_AKTL),
              threadIdx.x);
    lds_sync();
  }
  for (; it < items; it += gridDim.x) {
    const int nx = it + (int)gridDim.x;
    chunk_body<GATE, VEC_B, false, true>(q, k, v, vnew, dO, dR, g, beta, bgate, wgate, akk, hst, dhst, dq_out,
                                         dk_out, dv_out, dg_out, dbeta_out, db_out, dw_out, T, H, scale,
                                         nullptr, nullptr, nullptr, nullptr, 0, it, nx < items ? nx : -1, regA,
                                         regB, small, xbuf, gbuf, pin, nullptr, beta_sig, HQ);
  }
}

template <bool VEC_B, bool MAP = false>
__global__ __launch_bounds__(512) void matrix_intra_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const float* __restrict__ g,
    const float* __restrict__ beta, const bf16* __restrict__ bgate, const float* __restrict__ daqk,
    const float* __restrict__ dakk, float* __restrict__ dq, float* __restrict__ dk,
    float* __restrict__ db, float* __restrict__ dg, int T, int H, int beta_complete, int HQ,
    const int* __restrict__ cu, const int* __restrict__ ci) {
  using LY = PostLayout<CG_VECTOR, VEC_B, true>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PhaseIn pin;
  chunk_body<CG_VECTOR, VEC_B, true, false, -1, false, false, MAP>(
      q, k, nullptr, nullptr, nullptr, nullptr, g, beta, bgate, nullptr, dakk, nullptr, nullptr, nullptr, nullptr,
      nullptr, dg, VEC_B ? nullptr : db, nullptr, nullptr, T, H, 1.f, daqk, dq, dk, VEC_B ? db : nullptr,
      beta_complete, blockIdx.x, -1, smem, smem + LY::REGION_A,
      reinterpret_cast<float*>(smem + LY::REGION_A + LY::REGION_B), nullptr, nullptr, pin, nullptr, 0.f, HQ, cu, ci);
}

// Per-device, once: raise a kernel's dynamic-LDS limit (the attribute is held per
// device).  The flags are atomics: concurrent first calls from several host threads may
// both set the attribute (idempotent), and neither reads a torn flag.
constexpr int kMaxDevices = 64;
using LdsFlags = std::atomic<bool>[kMaxDevices];
static hipError_t allow_dynamic_lds(const void* kern, int bytes, LdsFlags& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  if (!done[dev].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    done[dev].store(true, std::memory_order_release);
  }
  return hipSuccess;
}

// compute units of the current device (cached per device)
static hipError_t device_cus(int& cus) {
  static std::atomic<int> cached[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (n <= 0) return hipErrorInvalidDevice;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  cus = n;
  return hipSuccess;
}

template <int GATE, bool VEC_B, bool HVF = false>
static hipError_t launch_post(const void* q, const void* k, const void* v, const void* vnew,
                              const void* dO, const void* dR, const float* g, const float* beta,
                              const void* bgate, const void* wgate, const float* akk, const void* h,
                              const void* dh, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                              void* db, void* dw, int B, int T, int H, int HQ, float scale, float beta_sig,
                              hipStream_t s, const int* cu = nullptr, const int* ci = nullptr) {
  const int items = B * H * (T / C);
  using LP = PostLayout<GATE, VEC_B, false, true>;
  using LY = PostLayout<GATE, VEC_B>;
  if (cu) {
    // a packed variable-length batch (sequences starting anywhere): the plain kernel
    auto kern = chunk_bwd_kernel<GATE, VEC_B, HVF, true>;
    static LdsFlags attr_set = {};
    const hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(items), dim3(512), LY::BYTES, s, (const bf16*)q, (const bf16*)k,
                       (const bf16*)v, (const bf16*)vnew, (const bf16*)dO, (const bf16*)dR, g, beta,
                       (const bf16*)bgate, (const bf16*)wgate, akk, (const bf16*)h, (const bf16*)dh,
                       (bf16*)dq, (bf16*)dk, (bf16*)dv, dg, dbeta, (bf16*)db, (bf16*)dw, T, H, scale, beta_sig, HQ,
                       cu, ci);
    return hipGetLastError();
  }
  // persistent form for scalar / no gate (measured slower for KDA: see the kernel)
  if constexpr (!HVF && LP::FITS && REWY_CHUNK_PIPE && (GATE != CG_VECTOR || REWY_CHUNK_PIPE > 1)) {
    auto kern = chunk_bwd_pipe_kernel<GATE, VEC_B>;    // static LDS only
    int cus = 0;
    const hipError_t e = device_cus(cus);
    if (e != hipSuccess) return e;
    const int grid = items < cus ? items : cus;        // one work-group per CU (LDS-bound)
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 0, s, (const bf16*)q, (const bf16*)k,
                       (const bf16*)v, (const bf16*)vnew, (const bf16*)dO, (const bf16*)dR, g, beta,
                       (const bf16*)bgate, (const bf16*)wgate, akk, (const bf16*)h, (const bf16*)dh,
                       (bf16*)dq, (bf16*)dk, (bf16*)dv, dg, dbeta, (bf16*)db, (bf16*)dw, T, H, scale, items,
                       beta_sig, HQ);
    return hipGetLastError();
  }
  auto kern = chunk_bwd_kernel<GATE, VEC_B, HVF>;
  static LdsFlags attr_set = {};
  const hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set);
  if (e != hipSuccess) return e;
  const int grid = items;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(512), LY::BYTES, s, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, (const bf16*)vnew, (const bf16*)dO, (const bf16*)dR, g, beta,
                     (const bf16*)bgate, (const bf16*)wgate, akk, (const bf16*)h, (const bf16*)dh,
                     (bf16*)dq, (bf16*)dk, (bf16*)dv, dg, dbeta, (bf16*)db, (bf16*)dw, T, H, scale, beta_sig, HQ,
                     nullptr, nullptr);
  return hipGetLastError();
}

}  // namespace rewy

using namespace rewy;

// B rows of T tokens, or (cu, ci) a packed batch of T / 64 chunks
static hipError_t chunk_bwd_dispatch(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                     const void* dR, const float* g, int gate_mode, const float* beta,
                                     const void* b_gate, const void* w_gate, const float* Akk, const void* h,
                                     const void* dh, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                                     float beta_sigmoid, void* db, void* dw, int h_v_first, int B, int T, int H,
                                     int qk_heads, float scale, hipStream_t stream, const int* cu, const int* ci) {
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ || (b_gate && HQ != H)) return hipErrorInvalidValue;
  if (!(beta_sigmoid >= 0.f) || (beta_sigmoid > 0.f && b_gate)) return hipErrorInvalidValue;
  if (!q || !k || !v || !v_new || !dO || !dR || !Akk || !h || !dh || !dq || !dk || !dv)
    return hipErrorInvalidValue;
  const bool vec_b = b_gate != nullptr;
  if (vec_b && (!w_gate || !db || !dw)) return hipErrorInvalidValue;
  if (!vec_b && (!beta || !dbeta)) return hipErrorInvalidValue;
  if (gate_mode != CG_NONE && (!g || !dg)) return hipErrorInvalidValue;
  if (vec_b && gate_mode != CG_VECTOR) return hipErrorInvalidValue;
#define FDR_POST(G, VB, HV)                                                                     \
  return launch_post<G, VB, HV>(q, k, v, v_new, dO, dR, g, beta, b_gate, w_gate, Akk, h, dh, dq, dk, \
                                dv, dg, dbeta, db, dw, B, T, H, HQ, scale, beta_sigmoid, stream, cu, ci)
  if (h_v_first) {
    // [V,K] states come from a saved forward: the vector-gate families (full saving)
    if (gate_mode != CG_VECTOR) return hipErrorInvalidValue;
    if (vec_b) { FDR_POST(CG_VECTOR, true, true); }
    FDR_POST(CG_VECTOR, false, true);
  }
  if (vec_b) { FDR_POST(CG_VECTOR, true, false); }
  switch (gate_mode) {
    case CG_NONE: FDR_POST(CG_NONE, false, false);
    case CG_SCALAR: FDR_POST(CG_SCALAR, false, false);
    case CG_VECTOR: FDR_POST(CG_VECTOR, false, false);
    default: return hipErrorInvalidValue;
  }
#undef FDR_POST
}

extern "C" hipError_t fdr_chunk_bwd(const void* q, const void* k, const void* v, const void* v_new,
                                    const void* dO, const void* dR, const float* g, int gate_mode,
                                    const float* beta, const void* b_gate, const void* w_gate,
                                    const float* Akk, const void* h, const void* dh, void* dq,
                                    void* dk, void* dv, float* dg, float* dbeta, float beta_sigmoid,
                                    void* db, void* dw, int h_v_first, int B, int T, int H, int qk_heads,
                                    int K, int V, int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0)
    return hipErrorInvalidValue;
  return chunk_bwd_dispatch(q, k, v, v_new, dO, dR, g, gate_mode, beta, b_gate, w_gate, Akk, h, dh, dq, dk, dv, dg,
                            dbeta, beta_sigmoid, db, dw, h_v_first, B, T, H, qk_heads, scale, stream, nullptr,
                            nullptr);
}

template <bool VEC_B, bool HVF, bool MAP>
static hipError_t launch_wy(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                            const void* dR, const float* g, const float* beta, const void* b_gate,
                            const void* w_gate, const float* Akk, const void* h, const void* dh, float* dq,
                            float* dk, void* dv, float* dbeta, float* db, void* dw, float* dg, float* dA, int items,
                            int T, int H, int HQ, float scale, const int* cu, const int* ci, hipStream_t stream) {
  using LY = PostLayout<CG_VECTOR, VEC_B>;
  auto kern = chunk_bwd_wy_kernel<VEC_B, HVF, MAP>;
  static LdsFlags attr_set = {};
  const hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(items), dim3(512), LY::BYTES, stream, (const bf16*)q, (const bf16*)k, (const bf16*)v,
                     (const bf16*)v_new, (const bf16*)dO, (const bf16*)dR, g, beta, (const bf16*)b_gate,
                     (const bf16*)w_gate, Akk, (const bf16*)h, (const bf16*)dh, dq, dk, (bf16*)dv, dg, dbeta, db,
                     (bf16*)dw, dA, T, H, scale, HQ, cu, ci);
  return hipGetLastError();
}

// KDA (beta) or GDN2 (b_gate, w_gate) WY seam over B rows of T tokens, or (cu, ci) a packed
// batch of T / 64 chunks
static hipError_t wy_dispatch(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                              const void* dR, const float* g, const float* beta, const void* b_gate,
                              const void* w_gate, const float* Akk, const void* h, const void* dh, float* dq,
                              float* dk, void* dv, float* dbeta, float* db, void* dw, float* dg, float* dA,
                              int h_v_first, int B, int T, int H, int HQ, float scale, const int* cu, const int* ci,
                              hipStream_t stream) {
  if (T <= 0 || T % C || B <= 0 || H <= 0 || H % HQ) return hipErrorInvalidValue;
  if (!q || !k || !v || !v_new || !dO || !dR || !g || !Akk || !h || !dh || !dq || !dk || !dv || !dg || !dA)
    return hipErrorInvalidValue;
  const bool vb = b_gate != nullptr;
  if (vb ? (!w_gate || !db || !dw || HQ != H) : (!beta || !dbeta)) return hipErrorInvalidValue;
  const int items = B * H * (T / C);
#define W_ARGS q, k, v, v_new, dO, dR, g, beta, b_gate, w_gate, Akk, h, dh, dq, dk, dv, dbeta, db, dw, dg, dA, items, \
               T, H, HQ, scale, cu, ci, stream
#define W_MAP(VB, HV) return cu ? launch_wy<VB, HV, true>(W_ARGS) : launch_wy<VB, HV, false>(W_ARGS);
  if (vb) {
    if (h_v_first) W_MAP(true, true) else W_MAP(true, false)
  }
  if (h_v_first) W_MAP(false, true) else W_MAP(false, false)
#undef W_MAP
#undef W_ARGS
}

extern "C" hipError_t fdr_chunk_bwd_wy(const void* q, const void* k, const void* v, const void* v_new,
                                       const void* dO, const void* dR, const float* g, const float* beta,
                                       const float* Akk, const void* h, const void* dh, float* dq, float* dk,
                                       void* dv, float* dbeta, float* dg, float* dA, int h_v_first, int B, int T,
                                       int H, int qk_heads, int K, int V, int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C) return hipErrorInvalidValue;
  return wy_dispatch(q, k, v, v_new, dO, dR, g, beta, nullptr, nullptr, Akk, h, dh, dq, dk, dv, dbeta, nullptr,
                     nullptr, dg, dA, h_v_first, B, T, H, qk_heads > 0 ? qk_heads : H, scale, nullptr, nullptr, stream);
}

extern "C" hipError_t fdr_chunk_bwd_wy_varlen(const void* q, const void* k, const void* v, const void* v_new,
                                              const void* dO, const void* dR, const float* g, const float* beta,
                                              const float* Akk, const void* h, const void* dh, float* dq, float* dk,
                                              void* dv, float* dbeta, float* dg, float* dA, int h_v_first,
                                              const int* cu_seqlens, const int* chunk_indices, int num_chunks, int H,
                                              int qk_heads, int K, int V, int chunk, float scale,
                                              hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || num_chunks <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return wy_dispatch(q, k, v, v_new, dO, dR, g, beta, nullptr, nullptr, Akk, h, dh, dq, dk, dv, dbeta, nullptr,
                     nullptr, dg, dA, h_v_first, 1, num_chunks * C, H, qk_heads > 0 ? qk_heads : H, scale,
                     cu_seqlens, chunk_indices, stream);
}

extern "C" hipError_t fdr_gdn2_chunk_bwd_wy(const void* q, const void* k, const void* v, const void* v_new,
                                            const void* dO, const void* dR, const float* g, const void* b_gate,
                                            const void* w_gate, const float* Akk, const void* h, const void* dh,
                                            float* dq, float* dk, void* dv, float* db, void* dw, float* dg, float* dA,
                                            int h_v_first, int B, int T, int H, int K, int V, int chunk, float scale,
                                            hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || !b_gate) return hipErrorInvalidValue;
  return wy_dispatch(q, k, v, v_new, dO, dR, g, nullptr, b_gate, w_gate, Akk, h, dh, dq, dk, dv, nullptr, db, dw, dg,
                     dA, h_v_first, B, T, H, H, scale, nullptr, nullptr, stream);
}

extern "C" hipError_t fdr_gdn2_chunk_bwd_wy_varlen(const void* q, const void* k, const void* v, const void* v_new,
                                                   const void* dO, const void* dR, const float* g, const void* b_gate,
                                                   const void* w_gate, const float* Akk, const void* h,
                                                   const void* dh, float* dq, float* dk, void* dv, float* db,
                                                   void* dw, float* dg, float* dA, int h_v_first,
                                                   const int* cu_seqlens, const int* chunk_indices, int num_chunks,
                                                   int H, int K, int V, int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || !b_gate || num_chunks <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return wy_dispatch(q, k, v, v_new, dO, dR, g, nullptr, b_gate, w_gate, Akk, h, dh, dq, dk, dv, nullptr, db, dw, dg,
                     dA, h_v_first, 1, num_chunks * C, H, H, scale, cu_seqlens, chunk_indices, stream);
}

extern "C" hipError_t fdr_chunk_bwd_varlen(const void* q, const void* k, const void* v, const void* v_new,
                                           const void* dO, const void* dR, const float* g, int gate_mode,
                                           const float* beta, const void* b_gate, const void* w_gate,
                                           const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                                           void* dv, float* dg, float* dbeta, float beta_sigmoid, void* db,
                                           void* dw, int h_v_first, const int* cu_seqlens,
                                           const int* chunk_indices, int num_chunks, int H, int qk_heads, int K,
                                           int V, int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || num_chunks <= 0 || H <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return chunk_bwd_dispatch(q, k, v, v_new, dO, dR, g, gate_mode, beta, b_gate, w_gate, Akk, h, dh, dq, dk, dv, dg,
                            dbeta, beta_sigmoid, db, dw, h_v_first, 1, num_chunks * C, H, qk_heads, scale, stream,
                            cu_seqlens, chunk_indices);
}

namespace rewy {
// gates.hip: ddt_bias / dA_log as column sums of [nrows][HK] / [nrows][HK/K*G] partials
hipError_t kda_gate_partials_sum(const float* part_dt, const float* part_da, int nrows, int HK, int G, float* ddt,
                                 float* dA, hipStream_t s);
}  // namespace rewy

extern "C" size_t fdr_chunk_bwd_gate_workspace_bytes(int B, int T, int H) {
  if (B <= 0 || T <= 0 || T % C || H <= 0) return 0;
  const size_t nblk = (size_t)B * (T / C);
  return nblk * ((size_t)H * KD + 8 * (size_t)H) * sizeof(float);
}

static hipError_t gate_fold_launch(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                   const void* dR, const float* g, const float* beta, const float* Akk, const void* h,
                                   const void* dh, void* dq, void* dk, void* dv, float* dbeta, float beta_sigmoid,
                                   const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
                                   int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log,
                                   float* ddt_bias, void* workspace, int h_v_first, int B, int T, int H, int qk_heads,
                                   int K, int V, int chunk, float scale, hipStream_t stream,
                                   const int* cu = nullptr, const int* ci = nullptr) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ) return hipErrorInvalidValue;
  if (!q || !k || !v || !v_new || !dO || !dR || !g || !beta || !Akk || !h || !dh || !dq || !dk || !dv || !dbeta)
    return hipErrorInvalidValue;
  if (!g_raw || !dg_raw || !workspace || !(beta_sigmoid >= 0.f)) return hipErrorInvalidValue;
  const int mode = !has_lower_bound ? (A_log ? 0 : -1) : (A_log ? 1 : 2);
  if (mode < 0) return hipErrorInvalidValue;
  const int nblk = B * (T / C);
  // every partial below is written by the chunk kernel before the column sums read it:
  // the workspace needs no clearing
  float* part_dt = reinterpret_cast<float*>(workspace);
  float* part_da = part_dt + (size_t)nblk * H * KD;
  const GateFoldArgs gf{g_raw, A_log, dt_bias, lower_bound, dg_raw, part_dt, part_da};
  using LY = PostLayout<CG_VECTOR, false>;
  const int fold = 2 * mode + (raw_is_bf16 ? 1 : 0) + (h_v_first ? 6 : 0) + (cu ? 12 : 0);
  using KernT = decltype(&chunk_bwd_fold_kernel<0>);
#define FOLD_KERNS(HV, M)                                                                                     \
  chunk_bwd_fold_kernel<0, HV, M>, chunk_bwd_fold_kernel<1, HV, M>, chunk_bwd_fold_kernel<2, HV, M>,          \
      chunk_bwd_fold_kernel<3, HV, M>, chunk_bwd_fold_kernel<4, HV, M>, chunk_bwd_fold_kernel<5, HV, M>
  static const KernT kerns[24] = {FOLD_KERNS(false, false), FOLD_KERNS(true, false), FOLD_KERNS(false, true),
                                  FOLD_KERNS(true, true)};
#undef FOLD_KERNS
  const KernT kern = kerns[fold];
  static LdsFlags attr_set[24] = {};
  hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set[fold]);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(B * H * (T / C)), dim3(512), LY::BYTES, stream, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, (const bf16*)v_new, (const bf16*)dO, (const bf16*)dR, g, beta, Akk,
                     (const bf16*)h, (const bf16*)dh, (bf16*)dq, (bf16*)dk, (bf16*)dv, dbeta, T, H, scale, gf,
                     beta_sigmoid, HQ, cu, ci);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return kda_gate_partials_sum(part_dt, part_da, nblk, H * KD, 8, ddt_bias, dA_log, stream);
}

extern "C" hipError_t fdr_chunk_bwd_gate_fold(const void* q, const void* k, const void* v, const void* v_new,
                                              const void* dO, const void* dR, const float* g, const float* beta,
                                              const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                                              void* dv, float* dbeta, float beta_sigmoid, const void* g_raw,
                                              int raw_is_bf16, const float* A_log, const float* dt_bias,
                                              int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log,
                                              float* ddt_bias, void* workspace, int h_v_first, int B, int T, int H,
                                              int qk_heads, int K, int V, int chunk, float scale,
                                              hipStream_t stream) {
  return gate_fold_launch(q, k, v, v_new, dO, dR, g, beta, Akk, h, dh, dq, dk, dv, dbeta, beta_sigmoid, g_raw,
                          raw_is_bf16, A_log, dt_bias, has_lower_bound, lower_bound, dg_raw, dA_log, ddt_bias,
                          workspace, h_v_first, B, T, H, qk_heads, K, V, chunk, scale, stream);
}

extern "C" hipError_t fdr_chunk_bwd_gate_fold_varlen(
    const void* q, const void* k, const void* v, const void* v_new, const void* dO, const void* dR, const float* g,
    const float* beta, const float* Akk, const void* h, const void* dh, void* dq, void* dk, void* dv, float* dbeta,
    float beta_sigmoid, const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
    int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log, float* ddt_bias, void* workspace,
    int h_v_first, const int* cu_seqlens, const int* chunk_indices, int num_chunks, int H, int qk_heads, int K,
    int V, int chunk, float scale, hipStream_t stream) {
  if (num_chunks <= 0 || !cu_seqlens || !chunk_indices) return hipErrorInvalidValue;
  return gate_fold_launch(q, k, v, v_new, dO, dR, g, beta, Akk, h, dh, dq, dk, dv, dbeta, beta_sigmoid, g_raw,
                          raw_is_bf16, A_log, dt_bias, has_lower_bound, lower_bound, dg_raw, dA_log, ddt_bias,
                          workspace, h_v_first, 1, num_chunks * C, H, qk_heads, K, V, chunk, scale, stream,
                          cu_seqlens, chunk_indices);
}

template <bool VEC_B, bool MAP>
static hipError_t launch_intra(const void* q, const void* k, const float* g, const float* beta,
                               const void* bgate, const float* daqk, const float* dakk, float* dq,
                               float* dk, float* db, float* dg, int B, int T, int H, int HQ, int beta_complete,
                               const int* cu, const int* ci, hipStream_t s) {
  using LY = PostLayout<CG_VECTOR, VEC_B, true>;
  auto kern = matrix_intra_kernel<VEC_B, MAP>;
  static LdsFlags attr_set = {};
  const hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(B * H * (T / C)), dim3(512), LY::BYTES, s, (const bf16*)q, (const bf16*)k, g,
                     beta, (const bf16*)bgate, daqk, dakk, dq, dk, db, dg, T, H, beta_complete, HQ, cu, ci);
  return hipGetLastError();
}

static hipError_t intra_dispatch(const void* q, const void* k, const float* g, const float* beta,
                                 const void* b_gate, const float* dAqk, const float* dAkk, float* dq, float* dk,
                                 float* db, float* dg, int B, int T, int H, int HQ, int beta_complete,
                                 const int* cu, const int* ci, hipStream_t s) {
  if (H % HQ || (b_gate && HQ != H)) return hipErrorInvalidValue;
  if (!b_gate && !beta) return hipErrorInvalidValue;
#define I_ARGS q, k, g, beta, b_gate, dAqk, dAkk, dq, dk, db, dg, B, T, H, HQ, beta_complete, cu, ci, s
  if (b_gate) return cu ? launch_intra<true, true>(I_ARGS) : launch_intra<true, false>(I_ARGS);
  return cu ? launch_intra<false, true>(I_ARGS) : launch_intra<false, false>(I_ARGS);
#undef I_ARGS
}

extern "C" hipError_t fdr_matrix_intra(const void* q, const void* k, const float* g, const float* beta,
                                       const void* b_gate, const float* dAqk, const float* dAkk, float* dq,
                                       float* dk, float* db, float* dg, int B, int T, int H, int qk_heads, int K,
                                       int chunk, int beta_complete, hipStream_t stream) {
  if (K != KD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (!q || !k || !g || !dAqk || !dAkk || !dq || !dk || !db || !dg) return hipErrorInvalidValue;
  const int HQ = qk_heads > 0 ? qk_heads : H;
  return intra_dispatch(q, k, g, b_gate ? nullptr : beta, b_gate, dAqk, dAkk, dq, dk, db, dg, B, T, H, HQ,
                        b_gate ? 0 : beta_complete, nullptr, nullptr, stream);
}

extern "C" hipError_t fdr_matrix_intra_varlen(const void* q, const void* k, const float* g, const float* beta,
                                              const void* b_gate, const float* dAqk, const float* dAkk, float* dq,
                                              float* dk, float* db, float* dg, const int* cu_seqlens,
                                              const int* chunk_indices, int num_chunks, int H, int qk_heads, int K,
                                              int chunk, int beta_complete, hipStream_t stream) {
  if (K != KD || chunk != C || num_chunks <= 0 || H <= 0 || !cu_seqlens || !chunk_indices) return hipErrorInvalidValue;
  if (!q || !k || !g || !dAqk || !dAkk || !dq || !dk || !db || !dg) return hipErrorInvalidValue;
  const int HQ = qk_heads > 0 ? qk_heads : H;
  return intra_dispatch(q, k, g, b_gate ? nullptr : beta, b_gate, dAqk, dAkk, dq, dk, db, dg, 1, num_chunks * C, H,
                        HQ, b_gate ? 0 : beta_complete, cu_seqlens, chunk_indices, stream);
}

// ---------------------------------------------------------------------------
// fdr_chunk_bwd_gate_fold without a workspace argument, for callers that cannot
// allocate (code under HIP graph capture, serving loops that forbid hipMalloc):
// the per-chunk partials live in a file-scope device array of fixed size that every
// GPU the library runs on holds until the process ends.  Calls that overlap on one
// GPU share it and race; nothing in it needs clearing (the chunk kernel writes every
// partial before the column sums read it).
// ---------------------------------------------------------------------------
#include <mutex>

static __device__ __align__(256) char scratch[FDR_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex scratch_mu;
void* scratch_dev[rewy::kMaxDevices];   // the array's device address, per device

// Device address of `scratch` on the current device, looked up once per device
// (the array's host-side name is not a device address).
hipError_t scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= rewy::kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return hipSuccess;
}
}  // namespace

extern "C" hipError_t fdr_chunk_bwd_gate_fold_noalloc(
    const void* q, const void* k, const void* v, const void* v_new, const void* dO, const void* dR, const float* g,
    const float* beta, const float* Akk, const void* h, const void* dh, void* dq, void* dk, void* dv, float* dbeta,
    float beta_sigmoid, const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
    int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log, float* ddt_bias, int h_v_first, int B,
    int T, int H, int qk_heads, int K, int V, int chunk, float scale, hipStream_t stream) {
  const size_t need = fdr_chunk_bwd_gate_workspace_bytes(B, T, H);
  if (need == 0 || need > FDR_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
  void* ws = nullptr;
  const hipError_t e = scratch_ptr(&ws);
  if (e != hipSuccess) return e;
  return gate_fold_launch(q, k, v, v_new, dO, dR, g, beta, Akk, h, dh, dq, dk, dv, dbeta, beta_sigmoid, g_raw,
                          raw_is_bf16, A_log, dt_bias, has_lower_bound, lower_bound, dg_raw, dA_log, ddt_bias, ws,
                          h_v_first, B, T, H, qk_heads, K, V, chunk, scale, stream);
}

extern "C" hipError_t fdr_chunk_bwd_original(const void* q, const void* k, const void* v, const void* v_new,
                                             const void* dO, const void* dR, const float* g, const float* beta,
                                             const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                                             void* dv, float* dg, float* dbeta, int B, int T, int H, int K, int V,
                                             int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (!q || !k || !v || !v_new || !dO || !dR || !g || !beta || !Akk || !h || !dh || !dq || !dk || !dv || !dg ||
      !dbeta)
    return hipErrorInvalidValue;
  using LY = PostLayout<CG_VECTOR, false, false, false, true>;
  static_assert(LY::BYTES <= 160 * 1024, "LDS budget");
  auto kern = chunk_bwd_original_kernel<0>;
  static LdsFlags attr_set = {};
  hipError_t e = allow_dynamic_lds((const void*)kern, LY::BYTES, attr_set);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(B * H * (T / C)), dim3(512), LY::BYTES, stream, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, (const bf16*)v_new, (const bf16*)dO, (const bf16*)dR, g, beta, Akk,
                     (const bf16*)h, (const bf16*)dh, (bf16*)dq, (bf16*)dk, (bf16*)dv, dg, dbeta, T, H, scale);
  return hipGetLastError();
}
