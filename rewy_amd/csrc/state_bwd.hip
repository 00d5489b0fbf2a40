// Reverse inter-chunk state recurrence of the chunked delta-rule backward.
//
// Replaces FLA's chunk_gated_delta_rule_bwd_dhu (called at reference
// backends/backward.py:120-121 and inside chunk_kda_bwd) and ReWY's
// vector_state_gpu.state_kernel (kernels/vector_state_gpu.py:12-43).  Per
// (batch, head, value tile) and for chunk c = NT-1 .. 0:
//
//   dh_out[c] = dh                                   (bf16)
//   dR_c      = kg_c dh + dv_local_c                 (bf16),  dv_local_c = Aqk_c^T dO_c
//   dh        = diag(lambda_c) dh + scale qg_c^T dO_c - w_c^T dR_c
//
// and dh0 = dh at the end (fp32).  dh is a 128 x BV fp32 tile held in
// accumulator registers for the whole sequence; all contractions run on
// v_mfma_f32_16x16x32_bf16.  Per-chunk operands are staged in LDS row-major,
// as they sit in HBM (coalesced 16-byte loads, one ds_write_b128 per piece);
// the contractions over tokens read them transposed with ds_read_b64_tr_b16.
// Operands of the next chunk are fetched into registers while the current
// chunk computes.  qg / kg (and w) may instead be formed from the raw q / k (and
// Akk, beta | b) as each chunk is staged: fdr_state_bwd_raw_qk.
#include "rewy_amd.h"

#include "state_body.hpp"

namespace rewy {

template <int BV, int GATE, bool DV_FROM_AQK, int NW, bool MAP = false, bool INL = false, bool RAWQK = false,
          int FW = 0>
__global__ __launch_bounds__(64 * NW) void state_bwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ w,
    const float* __restrict__ g, const bf16* __restrict__ dO, const float* __restrict__ aqk,
    const bf16* __restrict__ dv, const float* __restrict__ dht, bf16* __restrict__ dh_out,
    bf16* __restrict__ dr_out, float* __restrict__ dh0, int T, int H, float scale,
    const int* __restrict__ chunk_off, int segs, int vf, int HQ, const int* __restrict__ cu,
    const float* __restrict__ beta = nullptr, const bf16* __restrict__ bgate = nullptr,
    const float* __restrict__ akk = nullptr) {
  __shared__ StateSmem<BV, GATE, DV_FROM_AQK, INL, FW> sm;
  state_bwd_body<BV, GATE, DV_FROM_AQK, NW, MAP, INL, RAWQK, FW>(sm, xcd_logical_block(), q, k, w, g, dO, aqk, dv,
                                                                 dht, dh_out, dr_out, dh0, T, H, scale, chunk_off,
                                                                 segs, vf, HQ, cu, beta, bgate, akk);
}

template <int BV, int GATE, bool AQK, bool INL = false, bool RAWQK = false, int FW = 0>
static hipError_t launch_state(const void* q, const void* k, const void* w, const float* g,
                               const void* dO, const float* aqk, const void* dv, const float* dht,
                               void* dh, void* dr, float* dh0, int B, int T, int H, float scale,
                               hipStream_t stream, const int* chunk_off, int segs = 0, int vf = 0, int HQ = 0,
                               const int* cu = nullptr, const float* beta = nullptr, const void* bg = nullptr,
                               const float* akk = nullptr) {
  const int rows = segs > 0 ? B * segs : B;
  const int grid = rows * H * (VD / BV);
  // (FW at 32-wide tiles: 8 waves; 16 under their 128-register cap spill)
  constexpr int NW = FW ? 8 : state_waves<BV>();
#define S_LAUNCH(MAP)                                                                                        \
  hipLaunchKernelGGL((state_bwd_kernel<BV, GATE, AQK, NW, MAP, INL, RAWQK, FW>), dim3(grid), dim3(64 * NW), 0,   \
                     stream, (const bf16*)q, (const bf16*)k, (const bf16*)w, g, (const bf16*)dO, aqk,              \
                     (const bf16*)dv, dht, (bf16*)dh, (bf16*)dr, dh0, T, H, scale, chunk_off, segs, vf,            \
                     HQ > 0 ? HQ : H, cu, beta, (const bf16*)bg, akk)
  if constexpr (RAWQK) S_LAUNCH(false);     // (dense rows only)
  else if (cu) S_LAUNCH(true);
  else S_LAUNCH(false);
#undef S_LAUNCH
  return hipGetLastError();
}

template <int GATE, bool AQK, bool INL = false, bool RAWQK = false, int FW = 0>
static hipError_t pick_bv(int bv, const void* q, const void* k, const void* w, const float* g,
                          const void* dO, const float* aqk, const void* dv, const float* dht,
                          void* dh, void* dr, float* dh0, int B, int T, int H, float scale,
                          hipStream_t s, const int* co, int vf, int HQ, const int* cu, const float* beta = nullptr,
                          const void* bg = nullptr, const float* akk = nullptr) {
#define S_BV(BV) \
  launch_state<BV, GATE, AQK, INL, RAWQK, FW>(q, k, w, g, dO, aqk, dv, dht, dh, dr, dh0, B, T, H, scale, s, co, 0, \
                                              vf, HQ, cu, beta, bg, akk)
  switch (bv) {
    case 16: return S_BV(16);
    case 32: return S_BV(32);
    case 64: return S_BV(64);
    default: return hipErrorInvalidValue;
  }
#undef S_BV
}

// Segmented form, step 1: each segment's map from its end state X to its start state,
// dh_start = P X + Q.  One work-group per (segment, head, half): 64 columns of P (the
// recurrence run from the identity, without source terms) and 64 columns of Q (run from
// zero, with them) side by side in one 128 x 128 fp32 state, so the two halves share
// every staged operand (kg, w once; qg, Aqk and the dO columns only feed Q's columns).
// The per-chunk arithmetic is state_bwd_kernel's; nothing per chunk is stored.  P goes to
// pbuf [rows*segs, H, K, K] and Q to qbuf [rows*segs, H, K, V].
template <int GATE, bool DV_FROM_AQK>
struct XferSmem {
  static constexpr int LDK = KD + 8;
  static constexpr int LDT = C + 8;
  bf16 k[C][LDK];
  bf16 q[C * KD];
  bf16 w[2][C * KD];       // per chunk parity (read by the update, after a step's last barrier)
  bf16 ah[C * C];          // Aqk rows [t][s], bf16
  bf16 dO[C * 64];         // the Q half's 64 value columns
  bf16 dhT[128][LDK];      // state^T: columns 0-63 of P's half, 64-127 of Q's
  bf16 drT[128][LDT];
  float lam[2][KD];        // per chunk parity, as w
};

template <int GATE, bool DV_FROM_AQK>
__global__ __launch_bounds__(512) void state_xfer_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ w,
    const float* __restrict__ g, const bf16* __restrict__ dO, const float* __restrict__ aqk,
    const bf16* __restrict__ dv, float* __restrict__ pbuf, float* __restrict__ qbuf, int T, int H, float scale,
    int segs) {
  using S = XferSmem<GATE, DV_FROM_AQK>;
  __shared__ S sm;
  constexpr int NTH = 512, CHV = 8, NPD = C * CHV;
  const int logical = xcd_logical_block();
  const int half = logical & 1;
  const int bh = logical >> 1;
  const int b = bh / H, h = bh % H;
  const int row = b / segs, sg = b % segs, NTr = T / C;
  const int c0 = row * NTr + sg * NTr / segs;
  const int NT = row * NTr + (sg + 1) * NTr / segs - c0;
  const int base = 64 * half;           // P columns base .. base + 63; Q (value) columns likewise
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int rt = wv;                    // key rows [16 rt, 16 rt + 16), all 8 column tiles
  f32x4 st[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = 16 * rt + 4 * (l >> 4) + r;
      st[j][r] = (j < 4 && kr == base + 16 * j + (l & 15)) ? 1.f : 0.f;
    }
  }
  const int drow = wv & 3, dct0 = 4 * (wv >> 2);    // dR: waves 0-3 P's columns, 4-7 Q's
  const bool dq_half = dct0 >= 4;
  u32x4 rk[2], rq[2], rw[2], rdo;
  f32x4 ra[2];
  float rg_last = 0.f, rg_tok[2];
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;

  auto load_chunk = [&](int c) {
    const size_t tok0 = (size_t)(c0 + c) * C;
    if constexpr (GATE == GATE_VECTOR) {
      rg_last = g[((tok0 + C - 1) * H + h) * KD + (tid & (KD - 1))];     // (every lane: static wait counts)
    } else if constexpr (GATE == GATE_SCALAR) {
#pragma unroll
      for (int i = 0; i < 2; ++i) rg_tok[i] = g[(tok0 + ((tid + NTH * i) >> 4)) * H + h];
      rg_last = g[(tok0 + C - 1) * H + h];
    }
    const size_t kofs = tok0 * rsk + (size_t)h * KD;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      const size_t o = kofs + (size_t)(p >> 4) * rsk + (p & 15) * 8;
      rk[i] = *reinterpret_cast<const u32x4*>(k + o);
      rq[i] = *reinterpret_cast<const u32x4*>(q + o);
      rw[i] = *reinterpret_cast<const u32x4*>(w + o);
      if constexpr (DV_FROM_AQK)
        ra[i] = *reinterpret_cast<const f32x4*>(
            tril_src(aqk + ((tok0 + (p >> 4)) * H + h) * C + (p & 15) * 4, p >> 4, p & 15));
    }
    rdo = *reinterpret_cast<const u32x4*>(dO + (tok0 + tid / CHV) * rsv + (size_t)h * VD + base + (tid % CHV) * 8);
  };
  auto stage_chunk = [&](int db) {
    if (tid < KD) sm.lam[db][tid] = GATE == GATE_NONE ? 1.f : fast_exp2(rg_last);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      const int t = p >> 4, ch = p & 15;
      u32x4 kq = rk[i], qq = rq[i];
      if constexpr (GATE == GATE_SCALAR) {
        kq = scale_bf16x8(kq, fast_exp2(rg_last - rg_tok[i]));
        qq = scale_bf16x8(qq, fast_exp2(rg_tok[i]));
      }
      *reinterpret_cast<u32x4*>(&sm.k[t][ch * 8]) = kq;
      store_tr_chunk<16>(sm.q, t, ch, qq);
      store_tr_chunk<16>(sm.w[db], t, ch, rw[i]);
      if constexpr (DV_FROM_AQK) {
        bf16x4 hi;                           // one bf16 Aqk, as the direct kernel
#pragma unroll
        for (int r = 0; r < 4; ++r) hi[r] = to_bf16(tril_elem(ra[i][r], t, 4 * ch + r));
        *reinterpret_cast<bf16x4*>(sm.ah + tr_off<8>(t, ch * 4)) = hi;
      }
    }
    static_assert(NPD == NTH, "one dO piece per thread");
    store_tr_chunk<CHV>(sm.dO, tid / CHV, tid % CHV, rdo);
  };

  if (NT > 0) load_chunk(NT - 1);
  for (int c = NT - 1; c >= 0; --c) {
    // no barrier: every tile written before the next one was last read before the previous
    // step's last barrier (nothing per chunk is stored), except w and lambda, which the update
    // reads after it and which have a buffer per chunk parity
    const int db = c & 1;
    stage_chunk(db);
    if (c > 0) load_chunk(c - 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = to_bf16(st[j][r]);
      *reinterpret_cast<bf16x4*>(&sm.dhT[16 * j + (l & 15)][16 * rt + 4 * (l >> 4)]) = v4;
    }
    lds_barrier();
    // qg^T dO for Q's column tiles
    f32x4 xq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 a = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.q, 32 * ks, 16 * rt), frag_tr<CHV>(sm.dO, 32 * ks, 16 * j), a);
      xq[j] = a;
    }
    // dR = kg [P | Q] + [0 | dv_local]
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int ct = dct0 + cc;
      f32x4 a = zero4();
      if (dq_half) {
        if constexpr (DV_FROM_AQK) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 bo = frag_tr<CHV>(sm.dO, 32 * ks, 16 * cc);
            a = mfma(frag_tr<8>(sm.ah, 32 * ks, 16 * drow), bo, a);
          }
        } else {
          const size_t tok0 = (size_t)(c0 + c) * C;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * drow + 4 * (l >> 4) + r;
            a[r] = to_f32(dv[(tok0 + t) * rsv + (size_t)h * VD + base + 16 * cc + (l & 15)]);
          }
        }
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        a = mfma(frag(&sm.k[16 * drow][32 * ks], S::LDK), frag(&sm.dhT[16 * ct][32 * ks], S::LDK), a);
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = to_bf16(a[r]);
      *reinterpret_cast<bf16x4*>(&sm.drT[16 * ct + (l & 15)][16 * drow + 4 * (l >> 4)]) = v4;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f32x4 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * rt + 4 * (l >> 4) + r;
        a[r] = -(st[j][r] * sm.lam[db][kr] + (j >= 4 ? scale * xq[j - 4][r] : 0.f));
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.w[db], 32 * ks, 16 * rt), frag(&sm.drT[16 * j][32 * ks], S::LDT), a);
      st[j] = -a;
    }
  }
  float* pdst = pbuf + (size_t)bh * KD * KD;
  float* qdst = qbuf + (size_t)bh * KD * VD;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = 16 * rt + 4 * (l >> 4) + r;
      const int col = base + 16 * (j & 3) + (l & 15);
      (j < 4 ? pdst : qdst)[kr * KD + col] = st[j][r];
    }
}

// Segmented form, step 2: per (row, head, 8 state columns), walk the row's segments
// from the last to the first: X (the state at the segment's end; dht or zero for the
// last) is written to xbuf[segment], then X <- P X + Q, the state at the segment's
// start; after the first segment X is the row's dh0.  fp32 throughout.  P is staged in
// LDS transposed (coalesced global reads, fetched one segment ahead into registers;
// lane r then reads P[r][k] from consecutive banks), X in LDS; thread (r, half) owns
// state row r and 4 of the 8 columns.  Narrow column blocks give B*H*16 work-groups:
// the chain's length is the number of segments, each step a 128 x 128 x 8 product.
constexpr int COMB_COLS = 8;
__global__ __launch_bounds__(256) void state_combine_kernel(const float* __restrict__ pbuf,
                                                            const float* __restrict__ qbuf,
                                                            const float* __restrict__ dht, float* __restrict__ xbuf,
                                                            float* __restrict__ dh0, int segs, int H, int vf) {
  __shared__ float pt[KD][KD + 1];      // P^T of the current segment (odd pitch: transposed writes spread over banks)
  __shared__ f32x4 xs[KD][COMB_COLS / 4];
  const int bh = blockIdx.x, row = bh / H, h = bh % H;
  const int tid = threadIdx.x, r = tid >> 1, hc = tid & 1;
  const int col = COMB_COLS * blockIdx.y + 4 * hc;
  // dht / dh0 are [K,V] or (vf, state_v_first) [V,K] per (row, head)
  f32x4 x = zero4();
  if (dht) {
    const float* d = dht + (size_t)bh * KD * VD;
    if (vf) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = d[(col + e) * KD + r];
    } else {
      x = *reinterpret_cast<const f32x4*>(d + r * VD + col);
    }
  }
  f32x4 pre[KD * KD / 4 / 256];
  auto fetch = [&](int sg) {
    const float* P = pbuf + (((size_t)row * segs + sg) * H + h) * KD * KD;
#pragma unroll
    for (int i = 0; i < KD * KD / 4 / 256; ++i) {     // lanes along rows of P
      const int p4 = tid + 256 * i;
      pre[i] = *reinterpret_cast<const f32x4*>(P + (size_t)(p4 >> 5) * KD + 4 * (p4 & 31));
    }
  };
  fetch(segs - 1);
  for (int sg = segs - 1; sg >= 0; --sg) {
    const size_t seg = ((size_t)row * segs + sg) * H + h;
    const size_t xo = (seg * KD + r) * VD + col;
    f32x4 acc = *reinterpret_cast<const f32x4*>(qbuf + xo);
#pragma unroll
    for (int i = 0; i < KD * KD / 4 / 256; ++i) {
      const int p4 = tid + 256 * i, pr = p4 >> 5, pc = 4 * (p4 & 31);
#pragma unroll
      for (int e = 0; e < 4; ++e) pt[pc + e][pr] = pre[i][e];
    }
    xs[r][hc] = x;
    *reinterpret_cast<f32x4*>(xbuf + xo) = x;
    __syncthreads();
    if (sg > 0) fetch(sg - 1);
#pragma unroll 16
    for (int kk = 0; kk < KD; ++kk) {
      const float p = pt[kk][r];
      const f32x4 xv = xs[kk][hc];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(p, xv[e], acc[e]);
    }
    __syncthreads();
    x = acc;
  }
  if (dh0) {
    float* d = dh0 + (size_t)bh * KD * VD;
    if (vf) {
#pragma unroll
      for (int e = 0; e < 4; ++e) d[(col + e) * KD + r] = x[e];
    } else {
      *reinterpret_cast<f32x4*>(d + r * VD + col) = x;
    }
  }
}

template <int GATE, bool AQK>
static hipError_t launch_segmented(const void* q, const void* k, const void* w, const float* g, const void* dO,
                                   const float* aqk, const void* dv, const float* dht, void* dh, void* dr,
                                   float* dh0, int B, int T, int H, float scale, int segs, int bv, float* ws,
                                   int vf, hipStream_t s) {
  const size_t n = (size_t)B * segs * H * KD * VD;
  float* pbuf = ws;
  float* qbuf = ws + n;
  float* xbuf = ws + 2 * n;
  hipError_t e;
  // 1. per-segment maps P, Q (two work-groups per segment-head)
  hipLaunchKernelGGL((state_xfer_kernel<GATE, AQK>), dim3(B * segs * H * 2), dim3(512), 0, s, (const bf16*)q,
                     (const bf16*)k, (const bf16*)w, g, (const bf16*)dO, aqk, (const bf16*)dv, pbuf, qbuf, T, H,
                     scale, segs);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // 2. end states of every segment, sequential over segments
  hipLaunchKernelGGL(state_combine_kernel, dim3(B * H, VD / COMB_COLS), dim3(256), 0, s, pbuf, qbuf, dht, xbuf, dh0,
                     segs, H, vf);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // 3. every segment from its end state: dh per chunk and dR
  switch (bv) {
    case 16: return launch_state<16, GATE, AQK>(q, k, w, g, dO, aqk, dv, xbuf, dh, dr, nullptr, B, T, H, scale, s,
                                                nullptr, segs);
    case 32: return launch_state<32, GATE, AQK>(q, k, w, g, dO, aqk, dv, xbuf, dh, dr, nullptr, B, T, H, scale, s,
                                                nullptr, segs);
    case 64: return launch_state<64, GATE, AQK>(q, k, w, g, dO, aqk, dv, xbuf, dh, dr, nullptr, B, T, H, scale, s,
                                                nullptr, segs);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rewy

using namespace rewy;

// Value-tile width: the narrowest at which one launch holds at most 256 work-groups (one
// round on the CUs; a second round doubles the step chain), 64 beyond.  Measured (KDA state
// recurrence, T = 4096): B*H <= 32 16-wide fastest (the shortest step chain), 33-64 32-wide
// (BH = 48: 160 us vs 248 at 16-wide), from 65 64-wide even with CUs left idle (BH = 72: 213 us vs
// 280 at 32-wide; BH = 200: 445 vs 580): a wider tile shares each chunk's qg / kg / w loads over
// more value columns.
static int default_bv(int B, int H) {
  const int bh = B * H;
  if (bh * 8 <= 256) return 16;
  if (bh * 4 <= 256) return 32;
  return 64;
}

// B rows of T tokens, (chunk_off) B sequences packed along T tokens on 64-token boundaries,
// or (chunk_off, cu) B sequences packed anywhere along the token axis, in T / 64 chunks
static hipError_t state_dispatch(const void* q, const void* k, const void* w, const float* g, int gate_mode,
                                 const void* dO, const float* aqk, const void* dv, const float* dht, void* dh,
                                 void* dr, float* dh0, int B, int T, int H, int K, int V, int chunk, float scale,
                                 int value_block, hipStream_t stream, const int* co, int vf, int HQ,
                                 const int* cu = nullptr) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0)
    return hipErrorInvalidValue;
  if (!q || !k || !w || !dO || !dh || !dr) return hipErrorInvalidValue;
  // neither Aqk nor dv: the scalar / no-gate families form Aqk in-kernel from the raw q / k
  const bool inl = aqk == nullptr && dv == nullptr;
  if (aqk && dv) return hipErrorInvalidValue;
  if (inl && gate_mode == GATE_VECTOR) return hipErrorInvalidValue;
  if (gate_mode != GATE_NONE && g == nullptr) return hipErrorInvalidValue;
  if (HQ <= 0) HQ = H;
  if (H % HQ) return hipErrorInvalidValue;
  if (cu && !co) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : default_bv(B, H);
  const bool from_aqk = aqk != nullptr;
#define S_ARGS bv, q, k, w, g, dO, aqk, dv, dht, dh, dr, dh0, B, T, H, scale, stream, co, vf, HQ, cu
  switch (gate_mode) {
    case GATE_NONE:
      if (inl) return pick_bv<GATE_NONE, true, true>(S_ARGS);
      return from_aqk ? pick_bv<GATE_NONE, true>(S_ARGS) : pick_bv<GATE_NONE, false>(S_ARGS);
    case GATE_SCALAR:
      if (inl) return pick_bv<GATE_SCALAR, true, true>(S_ARGS);
      return from_aqk ? pick_bv<GATE_SCALAR, true>(S_ARGS) : pick_bv<GATE_SCALAR, false>(S_ARGS);
    case GATE_VECTOR:
      return from_aqk ? pick_bv<GATE_VECTOR, true>(S_ARGS) : pick_bv<GATE_VECTOR, false>(S_ARGS);
    default:
      return hipErrorInvalidValue;
  }
#undef S_ARGS
}

extern "C" hipError_t fdr_state_bwd(const void* q, const void* k, const void* w, const float* g,
                                    int gate_mode, const void* dO, const float* aqk, const void* dv,
                                    const float* dht, void* dh, void* dr, float* dh0, int state_v_first,
                                    int B, int T, int H, int qk_heads, int K, int V, int chunk, float scale,
                                    int value_block, hipStream_t stream) {
  return state_dispatch(q, k, w, g, gate_mode, dO, aqk, dv, dht, dh, dr, dh0, B, T, H, K, V, chunk, scale,
                        value_block, stream, nullptr, state_v_first ? 1 : 0, qk_heads);
}

extern "C" hipError_t fdr_state_bwd_raw_qk(const void* q, const void* k, const void* w, const float* g,
                                           const float* beta, const void* b_gate, const float* Akk,
                                           const void* dO, const float* aqk, const float* dht, void* dh, void* dr,
                                           float* dh0, int state_v_first, int B, int T, int H, int qk_heads, int K,
                                           int V, int chunk, float scale, int value_block, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (!q || !k || !g || !dO || !aqk || !dh || !dr) return hipErrorInvalidValue;
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : default_bv(B, H);
  const int vf = state_v_first ? 1 : 0;
  if (w) return pick_bv<GATE_VECTOR, true, false, true>(bv, q, k, w, g, dO, aqk, nullptr, dht, dh, dr, dh0, B, T, H,
                                                       scale, stream, nullptr, vf, HQ, nullptr);
  // w formed in-kernel from Akk and beta (scalar per row) or b_gate (GDN2, [B,T,H,K])
  if (!Akk || (beta == nullptr) == (b_gate == nullptr) || (b_gate && HQ != H)) return hipErrorInvalidValue;
  if (b_gate)
    return pick_bv<GATE_VECTOR, true, false, true, 2>(bv, q, k, nullptr, g, dO, aqk, nullptr, dht, dh, dr, dh0, B, T,
                                                      H, scale, stream, nullptr, vf, HQ, nullptr, nullptr, b_gate, Akk);
  return pick_bv<GATE_VECTOR, true, false, true, 1>(bv, q, k, nullptr, g, dO, aqk, nullptr, dht, dh, dr, dh0, B, T, H,
                                                    scale, stream, nullptr, vf, HQ, nullptr, beta, nullptr, Akk);
}

extern "C" hipError_t fdr_state_bwd_varlen(const void* q, const void* k, const void* w, const float* g,
                                           int gate_mode, const void* dO, const float* aqk, const void* dv,
                                           const float* dht, void* dh, void* dr, float* dh0, int state_v_first,
                                           const int* chunk_offsets, const int* cu_seqlens, int N, int num_chunks,
                                           int H, int qk_heads, int K, int V, int chunk, float scale,
                                           int value_block, hipStream_t stream) {
  if (!chunk_offsets || num_chunks <= 0) return hipErrorInvalidValue;
  return state_dispatch(q, k, w, g, gate_mode, dO, aqk, dv, dht, dh, dr, dh0, N, num_chunks * C, H, K, V, chunk,
                        scale, value_block, stream, chunk_offsets, state_v_first ? 1 : 0, qk_heads, cu_seqlens);
}

extern "C" size_t fdr_state_bwd_segmented_workspace_bytes(int B, int H, int segments) {
  if (B <= 0 || H <= 0 || segments <= 0) return 0;
  return 3 * (size_t)B * segments * H * KD * VD * sizeof(float);
}

extern "C" hipError_t fdr_state_bwd_segmented(const void* q, const void* k, const void* w, const float* g,
                                              int gate_mode, const void* dO, const float* aqk, const void* dv,
                                              const float* dht, void* dh, void* dr, float* dh0, int state_v_first,
                                              int B, int T, int H,
                                              int K, int V, int chunk, float scale, int segments, int value_block,
                                              void* workspace, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (!q || !k || !w || !dO || !dh || !dr || !workspace) return hipErrorInvalidValue;
  if ((aqk == nullptr) == (dv == nullptr)) return hipErrorInvalidValue;
  if (gate_mode != GATE_NONE && g == nullptr) return hipErrorInvalidValue;
  if (segments < 1 || segments > T / C) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : default_bv(B * segments, H);
  if (bv != 16 && bv != 32 && bv != 64) return hipErrorInvalidValue;
  float* ws = reinterpret_cast<float*>(workspace);
  const bool a = aqk != nullptr;
#define SEG_ARGS q, k, w, g, dO, aqk, dv, dht, dh, dr, dh0, B, T, H, scale, segments, bv, ws, state_v_first ? 1 : 0, stream
  switch (gate_mode) {
    case GATE_NONE: return a ? launch_segmented<GATE_NONE, true>(SEG_ARGS) : launch_segmented<GATE_NONE, false>(SEG_ARGS);
    case GATE_SCALAR:
      return a ? launch_segmented<GATE_SCALAR, true>(SEG_ARGS) : launch_segmented<GATE_SCALAR, false>(SEG_ARGS);
    case GATE_VECTOR:
      return a ? launch_segmented<GATE_VECTOR, true>(SEG_ARGS) : launch_segmented<GATE_VECTOR, false>(SEG_ARGS);
    default: return hipErrorInvalidValue;
  }
#undef SEG_ARGS
}
