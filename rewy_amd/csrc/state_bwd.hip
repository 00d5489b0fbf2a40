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
#include "common.hpp"
#include "rewy_amd.h"

namespace rewy {

enum GateMode { GATE_NONE = 0, GATE_SCALAR = 1, GATE_VECTOR = 2 };

template <int BV, int GATE, bool DV_FROM_AQK, bool INL = false, int FW = 0>
struct StateSmem {
  static constexpr int LDK = KD + 8;   // pitch of [.][K] tiles
  static constexpr int LDT = C + 8;    // pitch of [.][T] tiles
  static constexpr int CHV = BV / 8;   // 16-byte chunks per dO row
  // (INL at 64-wide tiles: k, q, Aqk and the row gates double-buffered by chunk parity -- see
  // the kernel)
  static constexpr bool SP = INL && BV == 64;
  static constexpr int NB = SP ? 2 : 1;
  // Outside SP the tiles a step's tail reads (dh^T for the stores, w and lambda for the
  // update) are double-buffered by chunk parity instead, so a step starts without a barrier
  static constexpr int ND = SP ? 1 : 2;
  bf16 k[NB][C][LDK];      // kg rows:  A operand of kg * dh           (contraction over K, row reads)
  bf16 q[NB][C * KD];      // qg rows:  A operand of qg^T dO           (over T, transposed reads)
  // (FW: w formed in-kernel between a step's two barriers, so one buffer)
  bf16 w[FW ? 1 : ND][C * KD];   // w rows: A operand of w^T dR      (over T, transposed reads)
  bf16 ah[NB][C * C];      // Aqk rows [t][s], bf16: A operand of Aqk^T dO (over T, transposed reads)
  bf16 dO[C * BV];         // dO rows [t][v]: B operand of both        (over T, transposed reads)
  bf16 dhT[ND][BV][LDK];   // dh^T:    B operand of kg * dh
  bf16 drT[BV][LDT];       // dR^T:    B operand of w^T dR
  float lam[ND][KD];       // exp2(g_last) per key row
  // in-kernel Aqk (INL, scalar / no gate): k and q are staged raw; qg^T dO is formed as
  // q^T (2^g dO) and kg dh as 2^(g_last - g_t) (k dh)
  bf16 dOg[(INL && GATE == GATE_SCALAR) ? C * BV : 1];   // 2^(g_t) dO rows (swizzled)
  float gt[NB][INL ? C + 1 : 1];                         // g_t per row, g_last at [C]
  // FW: E = (b k) 2^g rows (swizzled) and Akk hi / lo, the operands of w^T = E^T Akk^T
  // (16-byte aligned: they follow the 2- and 4-byte scalars above, and a 16-byte LDS read
  // from an address that is not measured 4x slower over the whole recurrence)
  alignas(16) bf16 e[FW ? C * KD : 1];
  alignas(16) bf16 akh[FW ? C : 1][LDT];
  alignas(16) bf16 akl[FW ? C : 1][LDT];
};

// NW waves: 8 (wave w owns state rows [16 w, 16 w + 16), every value column) or 16
// (row tile w % 8, half of the value columns).
//
// INL (scalar / no gate, with DV_FROM_AQK): Aqk = scale tril(q k^T 2^(g_i - g_s)) is formed
// in-kernel from the raw q / k each chunk stages anyway, instead of being read from HBM
// (fdr_prepare_wu then need not write it), and held as one bf16 for Aqk^T dO, as the
// reference's call for these families (FLA chunk_bwd_dv_local) rounds it.
//
// Segmented form (segs > 0): row r of T tokens is split into `segs` segments of
// consecutive chunks, work-group row b is segment b % segs of row b / segs, and dht holds
// each segment's end state (from state_combine_kernel).
// RAWQK (vector gate, dense rows): q and k are the raw ones (q/k heads HQ), and qg = q 2^g,
// kg = k 2^(g_last - g) are formed while the chunk is staged, with fdr_prepare_wu's roundings,
// from the gate tile the chunk loads beside them, so no qg / kg need be written for this pass.
// FW (with RAWQK; 1: scalar beta, 2: GDN2's vector b): w is not read either but formed as
// fdr_prepare_wu forms it, w^T = E^T Akk^T with E = (b k) 2^g and Akk split bf16 hi + lo, the
// same MFMA sequence and roundings, between the step's two barriers.
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
  static_assert(!INL || (DV_FROM_AQK && GATE != GATE_VECTOR), "in-kernel Aqk: scalar / no gate");
  static_assert(!RAWQK || (GATE == GATE_VECTOR && !INL && !MAP), "raw q / k: the vector gate, dense rows");
  static_assert(!FW || RAWQK, "w formed in-kernel: with the raw q / k");
  using S = StateSmem<BV, GATE, DV_FROM_AQK, INL, FW>;
  __shared__ S sm;
  constexpr int NVT = VD / BV;
  constexpr int NCT = BV / 16;             // column tiles of the state
  const int logical = xcd_logical_block();
  const int vt = logical % NVT;
  const int bh = logical / NVT;
  const int b = bh / H, h = bh % H;
  // chunks [c0, c0 + NT) of the packed token axis: row b of T tokens, segment b of the
  // segmented form, or sequence b of a variable-length batch (chunk_off: cumulative chunk
  // counts; clamped to the T / C chunks there are, an empty sequence passes its state through)
  int c0, NT;
  if (chunk_off) {
    c0 = min(max(chunk_off[b], 0), T / C);
    NT = max(min(chunk_off[b + 1], T / C) - c0, 0);
  } else if (segs > 0) {
    const int row = b / segs, sg = b % segs, NTr = T / C;
    c0 = row * NTr + sg * NTr / segs;
    NT = row * NTr + (sg + 1) * NTr / segs - c0;
  } else {
    c0 = b * (T / C);
    NT = T / C;
  }
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int v_base = vt * BV;

  // ---- state accumulators: wave wv owns key rows [16 rt, 16 rt + 16), column tiles ct0 .. ----
  constexpr int NTH = 64 * NW;
  constexpr int CG = NW / 8;                // waves per row tile
  constexpr int NCW = NCT / CG;             // column tiles per wave
  static_assert(NCW >= 1, "value tile too narrow for the wave count");
  const int rt = wv % 8, ct0 = NCW * (wv / 8);
  f32x4 st[NCW];
#pragma unroll
  for (int j = 0; j < NCW; ++j) {
    f32x4 a = zero4();
    if (dht) {
      const float* init = dht + (size_t)bh * KD * VD;
      const int col = v_base + 16 * (ct0 + j) + (l & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * rt + 4 * (l >> 4) + r;
        a[r] = init[vf ? col * KD + kr : kr * VD + col];     // [K,V] or, state_v_first, [V,K]
      }
    }
    st[j] = a;
  }
  // dR tiles: wave wv owns row tile (wv & 3) and column tiles [DCT * (wv >> 2), DCT * (wv >> 2) + DCT)
  constexpr int DCT = 4 * NCT >= NW ? 4 * NCT / NW : 1;
  const int drow = wv & 3;
  const int dct0 = DCT * (wv >> 2);
  const bool has_dr = dct0 < NCT;

  // ---- register staging of one chunk's operands (lanes run along rows) ----
  // kg, qg, w rows:  1024 16-byte pieces each, NPI per thread
  // Aqk rows (fp32): 1024 16-byte pieces, NPI per thread
  // dO rows:         8 * BV pieces
  constexpr int NPI = 1024 / NTH;
  constexpr int CHV = S::CHV;
  constexpr int NPD = C * CHV;
  constexpr int NDO = (NPD + NTH - 1) / NTH;
  u32x4 rk[NPI], rq[NPI], rw[NPI], rdo[NDO];
  f32x4 ra[NPI];
  float rg_last = 0.f, rg_tok[NPI];             // scalar gate: last row, the rows this thread stages
  float rg_do[NDO];                             // INL, scalar gate: the gate of each dO piece's row
  f32x4 rgp0[NPI], rgp1[NPI], rgl0, rgl1;       // RAWQK: each piece's 8 gates, g_last of its 8 columns
  u32x4 rbx[NPI];                               // FW = 2: b pieces
  float rbs[NPI];                               // FW = 1: beta of each piece's row
  f32x4 rak[NPI];                               // FW: Akk pieces
  const size_t row_stride_k = (size_t)H * KD;   // elements between tokens
  const size_t row_stride_v = (size_t)H * VD;

  auto load_chunk = [&](int c) {
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    // gate first: its consumer (lambda) is the first thing staged.  Every lane issues the same
    // loads (clamped indices): a branch here would make the vector-memory wait counts lane-
    // dependent, and the wait before staging would then fall to vmcnt(0) -- waiting also for
    // the previous step's dh / dR stores, issued after these loads
    if constexpr (GATE == GATE_VECTOR) {
      rg_last = g[((tok0 + rs_.clamp(C - 1)) * H + h) * KD + (tid & (KD - 1))];
    } else if constexpr (GATE == GATE_SCALAR) {
#pragma unroll
      for (int i = 0; i < NPI; ++i) rg_tok[i] = g[(tok0 + rs_.clamp((tid + NTH * i) >> 4)) * H + h];
      rg_last = g[(tok0 + rs_.clamp(C - 1)) * H + h];
    }
    const size_t kofs = tok0 * row_stride_k + (size_t)h * KD;
    // q / k: raw (HQ heads, grouped value heads) for scalar / no gates and RAWQK, qg / kg
    // (HQ = H) else
    const QKRows qr = qk_rows(tok0, h, H, HQ);
    if constexpr (RAWQK) {
      const float* gl = g + kofs + (size_t)rs_.clamp(C - 1) * row_stride_k + 8 * (tid & 15);
      rgl0 = *reinterpret_cast<const f32x4*>(gl);
      rgl1 = *reinterpret_cast<const f32x4*>(gl + 4);
#pragma unroll
      for (int i = 0; i < NPI; ++i) {
        const int p = tid + NTH * i;
        const float* gp = g + kofs + (size_t)rs_.clamp(p >> 4) * row_stride_k + (p & 15) * 8;
        rgp0[i] = *reinterpret_cast<const f32x4*>(gp);
        rgp1[i] = *reinterpret_cast<const f32x4*>(gp + 4);
      }
    }
#pragma unroll
    for (int i = 0; i < NPI; ++i) {
      const int p = tid + NTH * i;
      const size_t o = kofs + (size_t)(p >> 4) * row_stride_k + (p & 15) * 8;
      const size_t oq = qr.ofs + (size_t)(p >> 4) * qr.rs + (p & 15) * 8;
      rk[i] = *reinterpret_cast<const u32x4*>(rs_.src(k + oq, p >> 4));
      rq[i] = *reinterpret_cast<const u32x4*>(rs_.src(q + oq, p >> 4));
      if constexpr (FW) {
        rak[i] = *reinterpret_cast<const f32x4*>(
            tril_src(rs_.src(akk + ((tok0 + (p >> 4)) * H + h) * C + (p & 15) * 4, p >> 4), p >> 4, p & 15));
        if constexpr (FW == 2) rbx[i] = *reinterpret_cast<const u32x4*>(rs_.src(bgate + o, p >> 4));
        else rbs[i] = *rs_.src(beta + (tok0 + (p >> 4)) * H + h, p >> 4);
      } else {
        rw[i] = *reinterpret_cast<const u32x4*>(rs_.src(w + o, p >> 4));
      }
      if constexpr (DV_FROM_AQK && !INL)
        ra[i] = *reinterpret_cast<const f32x4*>(
            tril_src(rs_.src(aqk + ((tok0 + (p >> 4)) * H + h) * C + (p & 15) * 4, p >> 4), p >> 4, p & 15));
    }
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      // every lane loads (clamped to a valid piece) so the wait counts stay static
      const int p = min(tid + NTH * i, NPD - 1);
      rdo[i] = *reinterpret_cast<const u32x4*>(
          rs_.src(dO + (tok0 + p / CHV) * row_stride_v + (size_t)h * VD + v_base + (p % CHV) * 8, p / CHV));
      if constexpr (INL && GATE == GATE_SCALAR) rg_do[i] = g[(tok0 + rs_.clamp(p / CHV)) * H + h];
    }
  };

  auto stage_chunk = [&](int db) {
    if constexpr (GATE == GATE_VECTOR) {
      if (tid < KD) sm.lam[db][tid] = fast_exp2(rg_last);
    } else if constexpr (GATE == GATE_SCALAR) {
      if (tid < KD) sm.lam[db][tid] = fast_exp2(rg_last);
    } else {
      if (tid < KD) sm.lam[db][tid] = 1.f;
    }
#pragma unroll
    for (int i = 0; i < NPI; ++i) {
      const int p = tid + NTH * i;
      const int t = p >> 4, ch = p & 15;
      u32x4 kq = rk[i], qq = rq[i];
      if constexpr (RAWQK) {
        // qg = q 2^g, kg = k 2^(g_last - g), rounded as fdr_prepare_wu rounds them
        const bf16x8 kx = __builtin_bit_cast(bf16x8, rk[i]), qx = __builtin_bit_cast(bf16x8, rq[i]);
        bf16x8 ko, qo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float gj = j < 4 ? rgp0[i][j] : rgp1[i][j - 4];
          const float glj = j < 4 ? rgl0[j] : rgl1[j - 4];
          qo[j] = to_bf16(to_f32(qx[j]) * fast_exp2(gj));
          ko[j] = to_bf16(to_f32(kx[j]) * fast_exp2(glj - gj));
        }
        kq = __builtin_bit_cast(u32x4, ko);
        qq = __builtin_bit_cast(u32x4, qo);
        if constexpr (FW) {
          // E = (b k) 2^g and Akk hi / lo, rounded as fdr_prepare_wu rounds them
          bf16x8 eh;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float gj = j < 4 ? rgp0[i][j] : rgp1[i][j - 4];
            const float be = FW == 2 ? to_f32(__builtin_bit_cast(bf16x8, rbx[i])[j]) : rbs[i];
            eh[j] = to_bf16(be * to_f32(kx[j]) * fast_exp2(gj));
          }
          store_tr_chunk<16>(sm.e, t, ch, __builtin_bit_cast(u32x4, eh));
          bf16x4 alo;
          const bf16x4 ahi = split_hi4(tril_piece(rak[i], t, ch), alo);
          *reinterpret_cast<bf16x4*>(&sm.akh[t][4 * ch]) = ahi;
          *reinterpret_cast<bf16x4*>(&sm.akl[t][4 * ch]) = alo;
        }
      }
      if constexpr (GATE == GATE_SCALAR) {
        // scalar gate: kg = k 2^(g_last - g_t), qg = q 2^(g_t), the row's factors from registers
        kq = scale_bf16x8(kq, fast_exp2(rg_last - rg_tok[i]));
        qq = scale_bf16x8(qq, fast_exp2(rg_tok[i]));
      }
      *reinterpret_cast<u32x4*>(&sm.k[0][t][ch * 8]) = kq;
      store_tr_chunk<16>(sm.q[0], t, ch, qq);
      if constexpr (!FW) store_tr_chunk<16>(sm.w[db], t, ch, rw[i]);
      if constexpr (DV_FROM_AQK) {
        // Aqk as one bf16, the precision of the reference's dv_local (FLA's dAv rounds A to
        // the dO dtype before its dot: kernels/kda_residual_npu_onchip.py:114-116)
        bf16x4 hi;
#pragma unroll
        for (int r = 0; r < 4; ++r) hi[r] = to_bf16(tril_elem(ra[i][r], t, 4 * ch + r));
        *reinterpret_cast<bf16x4*>(sm.ah[0] + tr_off<8>(t, ch * 4)) = hi;
      }
    }
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int p = tid + NTH * i;
      if (NPD % NTH == 0 || p < NPD) store_tr_chunk<CHV>(sm.dO, p / CHV, p % CHV, rdo[i]);
    }
  };


  // In-kernel Aqk (INL): two load / stage groups, A (a chunk's raw k, q and row gates, g_last
  // included) and B (w, dO and 2^g dO).  At 64-wide tiles (SP) group A is staged one step ahead
  // into the parity buffer the chunk will read, so that its S = q k^T tiles are formed in the
  // step before -- after that step's state update, beside its stores, off the dependent chain
  // (registers at the start of step c: B holds chunk c, A chunk c - 1).  Narrower tiles (16
  // waves at 32-wide ones) measured slower so: they stage both groups of chunk c at step c and
  // form its S tiles before its dR.
  constexpr bool SP = S::SP;
  auto load_A = [&](int c) {
    if constexpr (INL) {
      const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
      const size_t tok0 = rs_.tok0;
      if constexpr (GATE == GATE_SCALAR) {
#pragma unroll
        for (int i = 0; i < NPI; ++i) rg_tok[i] = g[(tok0 + rs_.clamp((tid + NTH * i) >> 4)) * H + h];
        rg_last = g[(tok0 + rs_.clamp(C - 1)) * H + h];
      }
      const QKRows qr = qk_rows(tok0, h, H, HQ);
#pragma unroll
      for (int i = 0; i < NPI; ++i) {
        const int p = tid + NTH * i;
        const size_t oq = qr.ofs + (size_t)(p >> 4) * qr.rs + (p & 15) * 8;
        rk[i] = *reinterpret_cast<const u32x4*>(rs_.src(k + oq, p >> 4));
        rq[i] = *reinterpret_cast<const u32x4*>(rs_.src(q + oq, p >> 4));
      }
    }
  };
  auto load_B = [&](int c) {
    if constexpr (INL) {
      const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
      const size_t tok0 = rs_.tok0;
      const size_t kofs = tok0 * row_stride_k + (size_t)h * KD;
#pragma unroll
      for (int i = 0; i < NPI; ++i) {
        const int p = tid + NTH * i;
        rw[i] = *reinterpret_cast<const u32x4*>(rs_.src(w + kofs + (size_t)(p >> 4) * row_stride_k + (p & 15) * 8, p >> 4));
      }
#pragma unroll
      for (int i = 0; i < NDO; ++i) {
        const int p = min(tid + NTH * i, NPD - 1);
        rdo[i] = *reinterpret_cast<const u32x4*>(
            rs_.src(dO + (tok0 + p / CHV) * row_stride_v + (size_t)h * VD + v_base + (p % CHV) * 8, p / CHV));
        if constexpr (GATE == GATE_SCALAR) rg_do[i] = g[(tok0 + rs_.clamp(p / CHV)) * H + h];
      }
    }
  };
  // group A of the registers' chunk into parity buffer `pb`: raw k and q, the row gates
  auto stage_A = [&](int pb) {
    if constexpr (INL) {
#pragma unroll
      for (int i = 0; i < NPI; ++i) {
        const int p = tid + NTH * i;
        const int t = p >> 4, ch = p & 15;
        if (ch == 0) sm.gt[pb][t] = GATE == GATE_SCALAR ? rg_tok[i] : 0.f;
        *reinterpret_cast<u32x4*>(&sm.k[pb][t][ch * 8]) = rk[i];
        store_tr_chunk<16>(sm.q[pb], t, ch, rq[i]);
      }
      if (tid == 0) sm.gt[pb][C] = GATE == GATE_SCALAR ? rg_last : 0.f;
    }
  };
  auto stage_B = [&](int db) {
    if constexpr (INL) {
#pragma unroll
      for (int i = 0; i < NPI; ++i) {
        const int p = tid + NTH * i;
        store_tr_chunk<16>(sm.w[db], p >> 4, p & 15, rw[i]);
      }
#pragma unroll
      for (int i = 0; i < NDO; ++i) {
        const int p = tid + NTH * i;
        if (NPD % NTH == 0 || p < NPD) {
          store_tr_chunk<CHV>(sm.dO, p / CHV, p % CHV, rdo[i]);
          if constexpr (GATE == GATE_SCALAR)
            store_tr_chunk<CHV>(sm.dOg, p / CHV, p % CHV, scale_bf16x8(rdo[i], fast_exp2(rg_do[i])));
        }
      }
    }
  };
  // Aqk = scale tril(q k^T 2^(g_i - g_s)) of the chunk in buffer `pb`, as S^T = k q^T tiles
  // (rows s, columns i), so that each lane's four rows s are four consecutive columns of Aqk's
  // row i (as the read form stages it); one bf16, as FLA's chunk_bwd_dv_local rounds A before
  // its dot with dO
  auto form_S = [&](int pb) {
    if constexpr (INL) {
#pragma unroll
      for (int tt = wv; tt < 16; tt += NW) {
        const int Is = tt >> 2, Ji = tt & 3;
        f32x4 a = zero4();
        if (Ji >= Is) {                      // wave-uniform: tiles above the diagonal are zero
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            a = mfma(frag(&sm.k[pb][16 * Is][32 * ks], S::LDK), frag_row<16>(sm.q[pb], 16 * Ji, 32 * ks), a);
        }
        const int i = 16 * Ji + (l & 15);
        const float gi = sm.gt[pb][i];
        bf16x4 hi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s_ = 16 * Is + 4 * (l >> 4) + r;
          const float f = GATE == GATE_SCALAR ? scale * fast_exp2(gi - sm.gt[pb][s_]) : scale;
          hi[r] = to_bf16(i >= s_ ? a[r] * f : 0.f);
        }
        *reinterpret_cast<bf16x4*>(sm.ah[pb] + tr_off<8>(i, 16 * Is + 4 * (l >> 4))) = hi;
      }
    }
  };

  // global stores of dh[c] and dR_c from the transposed LDS copies: per wave task a block of
  // 16 columns (dh rows k / dR rows t) by 32 value rows, 16-lane group g taking 8 of them
  // (two transposed reads per 16-byte piece; narrower tiles repeat a group's rows, with the
  // same data; waves beyond the tasks skip, wave-uniform).  The loop is entered with as many
  // stores (sink: to the sink page) issued after the first chunk's loads as each step issues
  // after the next chunk's: where every wave has a task (64-wide tiles), the vector-memory wait
  // counts are then the same on both paths into a step, so its staging waits only for its own
  // loads, not for the previous step's stores.  (Narrower tiles keep waves without a task: a
  // split of each task over more waves, to keep the counts static there, measured slower.)  (Sink stores: one 16-byte slot each, at
  // most 3 per step here, so that none overwrites another and is dropped.)
  static_assert((KD / 16) * (BV >= 32 ? BV / 32 : 1) <= 2 * NW && (C / 16) * (BV >= 32 ? BV / 32 : 1) <= NW,
                "at most 3 stores per step, one sink-page slot each");
  auto store_tiles = [&](int c, int db, bool sink) {
    constexpr int RB = BV / 8;                          // 8-row blocks of the value tile
    constexpr int RQ = RB >= 4 ? RB / 4 : 1;            // quads of them
    const int g4 = l >> 4;
    const size_t dh_base = ((size_t)(c0 + c) * H + h) * KD * VD;
    constexpr int NTK = (KD / 16) * RQ;
#pragma unroll
    for (int i = 0; i < (NTK + NW - 1) / NW; ++i) {
      const int tk = wv + NW * i;
      if (NTK % NW != 0 && tk >= NTK) break;
      const int kr0 = 16 * (tk % (KD / 16)), v0 = 8 * ((4 * (tk / (KD / 16)) + g4) % RB);
      const bf16x8 o = col8_tr(&sm.dhT[db][0][0], S::LDK, v0, kr0, l);
      bf16* dst = dh_out + dh_base + (size_t)(kr0 + (l & 15)) * VD + v_base + v0;
      *reinterpret_cast<bf16x8*>(sink ? reinterpret_cast<bf16*>(sink_page + 4 * i) : dst) = o;
    }
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    constexpr int NTR = (C / 16) * RQ;
#pragma unroll
    for (int i = 0; i < (NTR + NW - 1) / NW; ++i) {
      const int tk = wv + NW * i;
      if (NTR % NW != 0 && tk >= NTR) break;
      const int t = 16 * (tk % (C / 16)) + (l & 15), v0 = 8 * ((4 * (tk / (C / 16)) + g4) % RB);
      const bf16x8 o = col8_tr(&sm.drT[0][0], S::LDT, v0, t - (l & 15), l);
      bf16* dst = rs_.dst(dr_out + (tok0 + t) * row_stride_v + (size_t)h * VD + v_base + v0, t);
      *reinterpret_cast<bf16x8*>(sink ? reinterpret_cast<bf16*>(sink_page + 4 * ((NTK + NW - 1) / NW + i)) : dst) = o;
    }
  };

  if constexpr (SP) {
    if (NT > 0) {
      load_A(NT - 1);
      load_B(NT - 1);
      stage_A((NT - 1) & 1);
      load_A(NT > 1 ? NT - 2 : 0);
      lds_barrier();
      form_S((NT - 1) & 1);
    }
  } else if constexpr (INL) {
    if (NT > 0) {
      load_A(NT - 1);
      load_B(NT - 1);
    }
  } else {
    if (NT > 0) load_chunk(NT - 1);
  }
  if (NT > 0) store_tiles(NT - 1, 0, true);
  for (int c = NT - 1; c >= 0; --c) {
    const int pb = SP ? (c & 1) : 0;     // this chunk's k / q / Aqk / gate buffer
    const int db = S::ND == 2 ? (c & 1) : 0;   // and its dh^T / w / lambda buffer
    // SP: the previous chunk done with every LDS tile.  Otherwise every tile written before
    // the next barrier was last read before the previous chunk's last barrier, or has a
    // buffer of its own (dh^T, w, lambda), so no barrier is needed here.
    if constexpr (SP) lds_barrier();
    if constexpr (SP) {
      stage_B(0);                          // chunk c
      stage_A(pb ^ 1);                     // chunk c - 1 (the last step stages chunk 0 again)
      load_B(c > 0 ? c - 1 : 0);
      load_A(c > 1 ? c - 2 : 0);
    } else if constexpr (INL) {
      stage_B(db);
      stage_A(0);
      if (c > 0) {
        load_A(c - 1);
        load_B(c - 1);
      }
    } else {
      stage_chunk(db);
      if (c > 0) load_chunk(c - 1);          // prefetch; consumed next iteration
    }
    // dh (state at the end of chunk c) -> LDS, transposed, bf16
#pragma unroll
    for (int j = 0; j < NCW; ++j) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = to_bf16(st[j][r]);
      *reinterpret_cast<bf16x4*>(&sm.dhT[db][16 * (ct0 + j) + (l & 15)][16 * rt + 4 * (l >> 4)]) = v4;
    }
    lds_barrier();

    if constexpr (INL && !SP) {
      form_S(0);
      lds_barrier();
    }

    // FW: w^T = E^T Akk^T of chunk c (the MFMA sequence of fdr_prepare_wu), for the update
    // after the next barrier: wave w takes token tile w % 4 and 32 / NW key-row tiles, so that
    // it reads one token tile's Akk hi / lo fragments and the E fragments of its key rows
    if constexpr (FW) {
      constexpr int TPW = 32 / NW;
      const int tt = wv % 4;
      const bf16x8 ah0 = frag(&sm.akh[16 * tt][0], S::LDT), al0 = frag(&sm.akl[16 * tt][0], S::LDT);
      const bf16x8 ah1 = frag(&sm.akh[16 * tt][32], S::LDT), al1 = frag(&sm.akl[16 * tt][32], S::LDT);
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int row0 = 16 * (TPW * (wv / 4) + i);
        const bf16x8 x0 = frag_tr<16>(sm.e, 0, row0);
        const bf16x8 x1 = frag_tr<16>(sm.e, 32, row0);
        f32x4 acc = zero4();
        acc = mfma(x0, ah0, acc);
        acc = mfma(x0, al0, acc);
        acc = mfma(x1, ah1, acc);
        acc = mfma(x1, al1, acc);
        bf16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = to_bf16(acc[r]);
        *reinterpret_cast<bf16x4*>(sm.w[0] + tr_off<16>(16 * tt + (l & 15), row0 + 4 * (l >> 4))) = o;
      }
    }
    // X = qg^T dO (independent of dh)
    f32x4 xq[NCW];
#pragma unroll
    for (int j = 0; j < NCW; ++j) {
      f32x4 a = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.q[pb], 32 * ks, 16 * rt),
                 frag_tr<CHV>(INL && GATE == GATE_SCALAR ? sm.dOg : sm.dO, 32 * ks, 16 * (ct0 + j)), a);
      xq[j] = a;
    }
    // dR tiles: kg dh + Aqk^T dO (+ dv)
    if (has_dr) {
#pragma unroll
      for (int cc = 0; cc < DCT; ++cc) {
        const int ct = dct0 + cc;
        f32x4 a = zero4();
        if constexpr (DV_FROM_AQK) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 bo = frag_tr<CHV>(sm.dO, 32 * ks, 16 * ct);
            a = mfma(frag_tr<8>(sm.ah[pb], 32 * ks, 16 * drow), bo, a);
          }
        } else {
          const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * drow + 4 * (l >> 4) + r;
            a[r] = to_f32(*rs_.src(dv + (rs_.tok0 + t) * row_stride_v + (size_t)h * VD + v_base + 16 * ct + (l & 15), t));
          }
        }
        if constexpr (INL && GATE == GATE_SCALAR) {
          // kg dh = 2^(g_last - g_t) (k dh), row t = 16 drow + 4 (l >> 4) + r
          f32x4 b = zero4();
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            b = mfma(frag(&sm.k[pb][16 * drow][32 * ks], S::LDK), frag(&sm.dhT[db][16 * ct][32 * ks], S::LDK), b);
#pragma unroll
          for (int r = 0; r < 4; ++r) a[r] += b[r] * fast_exp2(sm.gt[pb][C] - sm.gt[pb][16 * drow + 4 * (l >> 4) + r]);
        } else {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            a = mfma(frag(&sm.k[pb][16 * drow][32 * ks], S::LDK), frag(&sm.dhT[db][16 * ct][32 * ks], S::LDK), a);
        }
        bf16x4 v4;
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = to_bf16(a[r]);
        *reinterpret_cast<bf16x4*>(&sm.drT[16 * ct + (l & 15)][16 * drow + 4 * (l >> 4)]) = v4;
      }
    }
    // (read before the barrier: without SP the next chunk's staging may overwrite the gates)
    const float lam_inl = INL && GATE == GATE_SCALAR ? fast_exp2(sm.gt[pb][C]) : 1.f;
    lds_barrier();

    // dh <- lambda * dh + scale * X - w^T dR   (accumulated negated: -a + w^T dR)
#pragma unroll
    for (int j = 0; j < NCW; ++j) {
      f32x4 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * rt + 4 * (l >> 4) + r;
        a[r] = -(st[j][r] * (INL ? lam_inl : sm.lam[db][kr]) + scale * xq[j][r]);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.w[FW ? 0 : db], 32 * ks, 16 * rt), frag(&sm.drT[16 * (ct0 + j)][32 * ks], S::LDT),
                 a);
      st[j] = -a;
    }
    if constexpr (SP) form_S(pb ^ 1);      // chunk c - 1's Aqk, beside the stores

    store_tiles(c, db, false);
  }

  if (dh0) {
    float* dst = dh0 + (size_t)bh * KD * VD;
#pragma unroll
    for (int j = 0; j < NCW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * rt + 4 * (l >> 4) + r, col = v_base + 16 * (ct0 + j) + (l & 15);
        dst[vf ? col * KD + kr : kr * VD + col] = st[j][r];
      }
  }
}

// Waves per state work-group: 16 for 32-wide value tiles (4 % faster for GDN2's
// 512 work-groups), 8 otherwise (16 measured within 2 % at 64-wide tiles; 16-wide
// tiles have one column tile per row tile).
template <int BV>
constexpr int state_waves() { return BV == 32 ? 16 : 8; }

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

// Value-tile width chosen so that the grid fills the chip: the recurrence is
// sequential over chunks, so parallelism is B*H*(V/BV) work-groups.
static int default_bv(int B, int H) {
  const int bh = B * H;
  if (bh * 2 >= 256) return 64;
  if (bh * 4 >= 256) return 32;
  return 16;
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
