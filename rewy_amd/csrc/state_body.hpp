// The reverse inter-chunk state recurrence's work-group body (state_bwd_kernel in
// state_bwd.hip, and the state half of the paired launch in paired.hip): one (batch, head,
// value tile) work-group given its logical block index and its LDS.
#pragma once
#include "common.hpp"

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
__device__ __forceinline__ void state_bwd_body(
    StateSmem<BV, GATE, DV_FROM_AQK, INL, FW>& sm, int logical, const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ w,
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
  constexpr int NVT = VD / BV;
  constexpr int NCT = BV / 16;             // column tiles of the state
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

}  // namespace rewy
