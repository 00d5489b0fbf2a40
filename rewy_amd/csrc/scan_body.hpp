// The forward scan's work-group body with w / u formed in the sweep (fwd_h_wy_kernel in
// recompute.hip, and the scan half of the paired launch in paired.hip): one (batch, head,
// value tile) work-group given its logical block index and its LDS.
#pragma once
#include "common.hpp"

namespace rewy {

enum GateModeR { RG_NONE = 0, RG_SCALAR = 1, RG_VECTOR = 2 };

// ------------------------------------------------------------------------------------------
// fdr_fwd_h_wy: fdr_prepare_wu's w / u folded into the fdr_fwd_h sweep (scalar / no gate)
// ------------------------------------------------------------------------------------------
// Each (batch, head, value tile) work-group forms, per chunk, w^T = E^T A^T (E = beta k 2^g,
// every k row) and u^T = Z^T A^T (Z = beta v, its own value tile) with the MFMA sequence of
// prepare_wu_kernel, so w and u are the bits that kernel writes; u stays in LDS and w is
// written once (each value tile stores 64 / NVT of its rows) for the backward's state pass.
// A chunk's w / u do not depend on the state: they are formed one chunk ahead, beside the
// scan's dependent chain, and the launch replaces two (u written and read back, k read twice).
template <int BV>
struct FwdWySmem {
  static constexpr int LDK = KD + 8;
  static constexpr int LDT = C + 8;
  bf16 w[2][C][LDK];       // w rows of chunks c, c + 1 (by parity): A operand of w h, stored from here
  bf16 u[2][C * BV];       // u rows (swizzled), chunks c, c + 1: read transposed in the accumulator layout
  bf16 k[2][C * KD];       // kg rows (swizzled), chunks c, c + 1: A operand of kg^T v_new
  bf16 e[C * KD];          // E = b k 2^g rows of chunk c + 1 (swizzled): w^T = E^T A^T
  bf16 hT[BV][LDK];        // h^T: B operand of w h
  bf16 vT[BV][LDT];        // v_new^T: B operand of kg^T v_new
  bf16 z[C * BV];          // Z = w_gate v rows of chunk c + 1, this value tile (swizzled)
  bf16 ah[C][LDT];         // A rows of chunk c + 1, bf16 hi and lo
  bf16 al[C][LDT];
  float lam[2][KD];
};

// WG (fdr_fwd_h_u): w is given (w_in, as fdr_prepare_wu wrote it) and only u is formed here;
// k is the raw k (a vector gate's kg = k 2^(g_last - g) formed here, rounded as
// prepare_wu_kernel rounds it), and nothing but h, v_new (and the final state) is written.
// NOST (fdr_fwd_h_u with w NULL): w, u and kg all formed here, and again only h, v_new (and
// the final state) written: no q read, no w / qg / kg stored.
// KGIN (WG, vector gate): k is kg as fdr_prepare_wu wrote it (one row per value head), read
// instead of formed -- at narrow value tiles, where every tile would form it again.
template <int BV, int GATE, bool VEC_B, bool MAP, bool WG = false, bool NOST = false, bool KGIN = false>
__device__ __forceinline__ void fwd_h_wy_body(
    FwdWySmem<BV>& sm, int logical, const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const float* __restrict__ h0,
    bf16* __restrict__ w_out, bf16* __restrict__ qg_out, bf16* __restrict__ kg_out, bf16* __restrict__ h_out,
    bf16* __restrict__ vnew_out, float* __restrict__ ht_out, int T, int H, const int* __restrict__ chunk_off,
    int vf, int HQ, const int* __restrict__ cu, const bf16* __restrict__ w_in = nullptr) {
  static_assert(!VEC_B || GATE == RG_VECTOR, "vector b / w_gate come with the vector gate (GDN2)");
  static_assert(!(WG && NOST), "w given or formed, not both");
  static_assert(!KGIN || (WG && GATE == RG_VECTOR), "kg read: the vector gate's u-only scan");
  constexpr bool VEC = GATE == RG_VECTOR;
  using S = FwdWySmem<BV>;
  constexpr int NVT = VD / BV;
  constexpr int NCT = BV / 16;
  constexpr int NTH = 512;
  constexpr int RW = C / NVT;          // rows of w (and qg, kg) this value tile stores
  const int vt = logical % NVT;
  const int bh = logical / NVT;
  const int b = bh / H, h = bh % H;
  const int c0 = chunk_off ? min(max(chunk_off[b], 0), T / C) : b * (T / C);
  const int NT = chunk_off ? max(min(chunk_off[b + 1], T / C) - c0, 0) : T / C;
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int lc = l & 15, lg = l >> 4;
  const int v_base = vt * BV;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;

  // state rows [16 wv, 16 wv + 16)
  f32x4 st[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    f32x4 a = zero4();
    if (h0) {
      const float* src = h0 + (size_t)bh * KD * VD;     // [K,V] or, state_v_first (vf), [V,K]
      const int col = v_base + 16 * ct + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * wv + 4 * lg + r;
        a[r] = src[vf ? col * KD + kr : kr * VD + col];
      }
    }
    st[ct] = a;
  }
  constexpr int DCT = NCT >= 2 ? NCT / 2 : 1;
  const int drow = wv & 3;
  const int dct0 = DCT * (wv >> 2);
  const bool has_dr = dct0 < NCT;

  // Pipeline: step c stages chunk c + 1 beside its v_new product and forms chunk c + 1's
  // w / u beside its state update and stores, off the scan's dependent chain; w, u, kg and
  // lambda are double-buffered by chunk parity.  Registers hold chunk c + 1's operands,
  // loaded one step ahead: per piece p = tid + 512 i (row p >> 4, columns 8 (p & 15) ..) the
  // k (, q, g, b) pieces and 4 A columns, the value tile's v (, w_gate) pieces, and the gate /
  // beta scalars of those rows.
  constexpr int CHV = BV / 8;
  constexpr int NPU = C * CHV;
  constexpr int NU = (NPU + NTH - 1) / NTH;
  u32x4 rk[2], rq[2], rb[2], rv[NU], rwg[NU];
  f32x4 ra[2], rg0[2], rg1[2], rgl0, rgl1;
  float rg_last = 0.f, rg_tok[2] = {0.f, 0.f}, rb_tok[2] = {0.f, 0.f}, rb_v[NU];
  auto load_chunk = [&](int c) {
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    const size_t kofs = tok0 * rsk + (size_t)h * KD;
    if constexpr (GATE == RG_SCALAR) {
#pragma unroll
      for (int i = 0; i < 2; ++i) rg_tok[i] = g[(tok0 + rs_.clamp((tid + NTH * i) >> 4)) * H + h];
      rg_last = g[(tok0 + rs_.clamp(C - 1)) * H + h];
    } else if constexpr (VEC) {
      // lambda's column (tid < KD), and g_last of this thread's 8 columns (both pieces)
      rg_last = g[kofs + (size_t)rs_.clamp(C - 1) * rsk + (tid & (KD - 1))];
      if constexpr (!KGIN) {
        const float* gl = g + kofs + (size_t)rs_.clamp(C - 1) * rsk + 8 * (tid & 15);
        rgl0 = *reinterpret_cast<const f32x4*>(gl);
        rgl1 = *reinterpret_cast<const f32x4*>(gl + 4);
      }
    }
    const QKRows kr_ = KGIN ? QKRows{kofs, rsk} : qk_rows(tok0, h, H, HQ);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i, t = p >> 4, c8 = 8 * (p & 15);
      if constexpr (WG) {
        rq[i] = *reinterpret_cast<const u32x4*>(rs_.src(w_in + kofs + (size_t)t * rsk + c8, t));   // w rows
        if constexpr (VEC && !KGIN) {
          rg0[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rs_.clamp(t) * rsk + c8);
          rg1[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rs_.clamp(t) * rsk + c8 + 4);
        }
      } else {
        if constexpr (VEC) {
          rg0[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rs_.clamp(t) * rsk + c8);
          rg1[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rs_.clamp(t) * rsk + c8 + 4);
          if constexpr (!NOST) rq[i] = *reinterpret_cast<const u32x4*>(rs_.src(q + kr_.ofs + (size_t)t * kr_.rs + c8, t));
        }
        if constexpr (VEC_B) rb[i] = *reinterpret_cast<const u32x4*>(rs_.src(bgate + kofs + (size_t)t * rsk + c8, t));
        else rb_tok[i] = *rs_.src(beta + (tok0 + t) * H + h, t);
      }
      rk[i] = *reinterpret_cast<const u32x4*>(rs_.src(k + kr_.ofs + (size_t)t * kr_.rs + c8, t));
      ra[i] = *reinterpret_cast<const f32x4*>(tril_src(rs_.src(akk + ((tok0 + t) * H + h) * C + 4 * (p & 15), t),
                                                       t, p & 15));
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int p = min(tid + NTH * i, NPU - 1), t = p / CHV;
      const size_t vo = (tok0 + t) * rsv + (size_t)h * VD + v_base + (p % CHV) * 8;
      if constexpr (VEC_B) rwg[i] = *reinterpret_cast<const u32x4*>(rs_.src(wgate + vo, t));
      else rb_v[i] = *rs_.src(beta + (tok0 + t) * H + h, t);
      rv[i] = *reinterpret_cast<const u32x4*>(rs_.src(v + vo, t));
    }
  };
  // the registers' chunk (c) into LDS: E, Z, A (hi / lo) for its w / u, kg and lambda into
  // buffer `pb`; vector gates also store its qg and kg rows of this value tile's share
  auto stage_chunk = [&](int pb, int c) {
    if (tid < KD) sm.lam[pb][tid] = GATE == RG_NONE ? 1.f : fast_exp2(rg_last);
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t kofs = rs_.tok0 * rsk + (size_t)h * KD;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      const int t = p >> 4, ch = p & 15;
      // E = (b k) 2^g and kg = k 2^(g_last - g), each rounded as prepare_wu_kernel rounds it
      const bf16x8 kx = __builtin_bit_cast(bf16x8, rk[i]);
      bf16x8 eh, kg;
      if constexpr (WG) {
        // w as given, kg formed (the scalar gate's as fdr_fwd_h forms it); no E
        *reinterpret_cast<u32x4*>(&sm.w[pb][t][8 * ch]) = rq[i];
        if constexpr (KGIN) {
          kg = kx;
        } else if constexpr (VEC) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float gj = j < 4 ? rg0[i][j] : rg1[i][j - 4];
            const float glj = j < 4 ? rgl0[j] : rgl1[j - 4];
            kg[j] = to_bf16(to_f32(kx[j]) * fast_exp2(glj - gj));
          }
        } else {
          kg = GATE == RG_SCALAR ? __builtin_bit_cast(bf16x8, scale_bf16x8(rk[i], fast_exp2(rg_last - rg_tok[i]))) : kx;
        }
      } else if constexpr (VEC) {
        const bf16x8 qx = NOST ? bf16x8{} : __builtin_bit_cast(bf16x8, rq[i]);
        bf16x8 bx = {};
        if constexpr (VEC_B) bx = __builtin_bit_cast(bf16x8, rb[i]);
        bf16x8 qg;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float gj = j < 4 ? rg0[i][j] : rg1[i][j - 4];
          const float glj = j < 4 ? rgl0[j] : rgl1[j - 4];
          const float be = VEC_B ? to_f32(bx[j]) : rb_tok[i];
          eh[j] = to_bf16(be * to_f32(kx[j]) * fast_exp2(gj));
          if constexpr (!NOST) qg[j] = to_bf16(to_f32(qx[j]) * fast_exp2(gj));
          kg[j] = to_bf16(to_f32(kx[j]) * fast_exp2(glj - gj));
        }
        if (!NOST && t / RW == vt) {       // (wave-uniform: a wave's 64 pieces are 4 whole rows)
          *reinterpret_cast<bf16x8*>(rs_.dst(qg_out + kofs + (size_t)t * rsk + 8 * ch, t)) = qg;
          *reinterpret_cast<bf16x8*>(rs_.dst(kg_out + kofs + (size_t)t * rsk + 8 * ch, t)) = kg;
        }
      } else {
        const float ge = GATE == RG_SCALAR ? fast_exp2(rg_tok[i]) : 1.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) eh[j] = to_bf16(rb_tok[i] * to_f32(kx[j]) * ge);
        kg = GATE == RG_SCALAR ? __builtin_bit_cast(bf16x8, scale_bf16x8(rk[i], fast_exp2(rg_last - rg_tok[i]))) : kx;
      }
      if constexpr (!WG) store_tr_chunk<16>(sm.e, t, ch, __builtin_bit_cast(u32x4, eh));
      store_tr_chunk<16>(sm.k[pb], t, ch, __builtin_bit_cast(u32x4, kg));
      bf16x4 alo;
      const bf16x4 ahi = split_hi4(tril_piece(ra[i], t, ch), alo);
      *reinterpret_cast<bf16x4*>(&sm.ah[t][4 * ch]) = ahi;
      *reinterpret_cast<bf16x4*>(&sm.al[t][4 * ch]) = alo;
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int p = tid + NTH * i;
      if (NPU % NTH == 0 || p < NPU) {
        const bf16x8 vx = __builtin_bit_cast(bf16x8, rv[i]);
        bf16x8 zh;
        if constexpr (VEC_B) {
          const bf16x8 wx = __builtin_bit_cast(bf16x8, rwg[i]);
#pragma unroll
          for (int j = 0; j < 8; ++j) zh[j] = to_bf16(to_f32(wx[j]) * to_f32(vx[j]));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) zh[j] = to_bf16(rb_v[i] * to_f32(vx[j]));
        }
        store_tr_chunk<CHV>(sm.z, p / CHV, p % CHV, __builtin_bit_cast(u32x4, zh));
      }
    }
  };
  // w^T = E^T A^T (wave wv: k rows [16 wv, 16 wv + 16), all 64 tokens) and u^T = Z^T A^T
  // ((value row tile, token tile) pairs over the waves) of the staged chunk, into buffer `pb`
  auto form_wu = [&](int pb) {
    if constexpr (!WG) {
      const int row0 = 16 * wv;
      const bf16x8 x0 = frag_tr<16>(sm.e, 0, row0);
      const bf16x8 x1 = frag_tr<16>(sm.e, 32, row0);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        f32x4 acc = zero4();
        acc = mfma(x0, frag(&sm.ah[16 * tt][0], S::LDT), acc);
        acc = mfma(x0, frag(&sm.al[16 * tt][0], S::LDT), acc);
        acc = mfma(x1, frag(&sm.ah[16 * tt][32], S::LDT), acc);
        acc = mfma(x1, frag(&sm.al[16 * tt][32], S::LDT), acc);
        bf16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = to_bf16(acc[r]);
        *reinterpret_cast<bf16x4*>(&sm.w[pb][16 * tt + lc][row0 + 4 * lg]) = o;
      }
    }
#pragma unroll
    for (int ut = wv; ut < NCT * 4; ut += 8) {
      const int rt = ut % NCT, tt = ut / NCT;
      const bf16x8 x0 = frag_tr<CHV>(sm.z, 0, 16 * rt);
      const bf16x8 x1 = frag_tr<CHV>(sm.z, 32, 16 * rt);
      f32x4 acc = zero4();
      acc = mfma(x0, frag(&sm.ah[16 * tt][0], S::LDT), acc);
      acc = mfma(x0, frag(&sm.al[16 * tt][0], S::LDT), acc);
      acc = mfma(x1, frag(&sm.ah[16 * tt][32], S::LDT), acc);
      acc = mfma(x1, frag(&sm.al[16 * tt][32], S::LDT), acc);
      bf16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = to_bf16(acc[r]);
      *reinterpret_cast<bf16x4*>(sm.u[pb] + tr_off<CHV>(16 * tt + lc, 16 * rt + 4 * lg)) = o;
    }
  };
  auto settle_chunk = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      settle(rk[i]);
      settle(ra[i]);
      if constexpr (WG) {
        settle(rq[i]);
        if constexpr (VEC && !KGIN) {
          settle(rg0[i]);
          settle(rg1[i]);
        }
      } else {
        if constexpr (VEC) {
          if constexpr (!NOST) settle(rq[i]);
          settle(rg0[i]);
          settle(rg1[i]);
        }
        if constexpr (VEC_B) settle(rb[i]);
        else settle(rb_tok[i]);
      }
      if constexpr (GATE == RG_SCALAR) settle(rg_tok[i]);
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      settle(rv[i]);
      if constexpr (VEC_B) settle(rwg[i]);
      else settle(rb_v[i]);
    }
    if constexpr (VEC && !KGIN) {
      settle(rgl0);
      settle(rgl1);
    }
    settle(rg_last);
  };
  if (NT > 0) {
    load_chunk(0);
    settle_chunk();
    stage_chunk(0, 0);
    load_chunk(NT > 1 ? 1 : 0);
    lds_barrier();
    form_wu(0);
    settle_chunk();
  }
  for (int c = 0; c < NT; ++c) {
    const int pb = c & 1;
    lds_barrier();
    // h_c -> LDS (transposed, bf16); the same rounded values feed w h, as stored
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = to_bf16(st[ct][r]);
      *reinterpret_cast<bf16x4*>(&sm.hT[16 * ct + lc][16 * wv + 4 * lg]) = v4;
    }
    lds_barrier();
    const int cn = c + 1 < NT ? c + 1 : c;   // (the last step stages itself again: no branch)
    stage_chunk(pb ^ 1, cn);
    load_chunk(c + 2 < NT ? c + 2 : NT - 1);
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    // w rows [64 vt / NVT, ...) of chunk c to HBM, 16-byte pieces (every lane stores: pieces
    // beyond the share are written twice, with the same data); WG: w came from HBM
    if constexpr (!WG && !NOST) {
      constexpr int NWP = RW * (KD / 8);
#pragma unroll
      for (int i = 0; i < (NWP + NTH - 1) / NTH; ++i) {
        const int p = (tid + NTH * i) % NWP;
        const int t = vt * RW + p / (KD / 8), c8 = 8 * (p % (KD / 8));
        *reinterpret_cast<u32x4*>(rs_.dst(w_out + (tok0 + t) * rsk + (size_t)h * KD + c8, t)) =
            *reinterpret_cast<const u32x4*>(&sm.w[pb][t][c8]);
      }
    }
    // v_new tiles = u - w h
    if (has_dr) {
#pragma unroll
      for (int cc = 0; cc < DCT; ++cc) {
        const int ct = dct0 + cc;
        const bf16x4 u4 =
            ds_read_tr4(sm.u[pb] + tr_off<CHV>(16 * drow + 4 * lg + (lc >> 2), 16 * ct + 4 * (lc & 3)));
        f32x4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = -to_f32(u4[r]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          a = mfma(frag(&sm.w[pb][16 * drow][32 * ks], S::LDK), frag(&sm.hT[16 * ct][32 * ks], S::LDK), a);
        bf16x4 v4;
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = to_bf16(-a[r]);
        *reinterpret_cast<bf16x4*>(&sm.vT[16 * ct + lc][16 * drow + 4 * lg]) = v4;
      }
    }
    lds_barrier();
    // h <- lambda h + kg^T v_new
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) a[r] = st[ct][r] * sm.lam[pb][16 * wv + 4 * lg + r];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.k[pb], 32 * ks, 16 * wv), frag(&sm.vT[16 * ct][32 * ks], S::LDT), a);
      st[ct] = a;
    }
    form_wu(pb ^ 1);                         // chunk c + 1's w / u, beside the update and the stores
    {
      const size_t hb = ((size_t)(c0 + c) * H + h) * KD * VD;
      // per wave task a block of 16 columns (h rows k / v_new rows t) by 32 value rows, 16-lane
      // group g taking 8 of them (two transposed reads per 16-byte piece)
      constexpr int RB = BV / 8, RQ = RB >= 4 ? RB / 4 : 1, NW = NTH / 64;
      constexpr int NTK = (KD / 16) * RQ, NTR = (C / 16) * RQ;
#pragma unroll
      for (int i = 0; i < (NTK + NW - 1) / NW; ++i) {
        const int tk = (wv + NW * i) % NTK;
        const int kr0 = 16 * (tk % (KD / 16)), v0 = 8 * ((4 * (tk / (KD / 16)) + (l >> 4)) % RB);
        const bf16x8 o = col8_tr(&sm.hT[0][0], S::LDK, v0, kr0, l);
        *reinterpret_cast<bf16x8*>(h_out + hb + (size_t)(kr0 + (l & 15)) * VD + v_base + v0) = o;
      }
#pragma unroll
      for (int i = 0; i < (NTR + NW - 1) / NW; ++i) {
        const int tk = (wv + NW * i) % NTR;
        const int t0 = 16 * (tk % (C / 16)), t = t0 + (l & 15), v0 = 8 * ((4 * (tk / (C / 16)) + (l >> 4)) % RB);
        const bf16x8 o = col8_tr(&sm.vT[0][0], S::LDT, v0, t0, l);
        *reinterpret_cast<bf16x8*>(rs_.dst(vnew_out + (tok0 + t) * rsv + (size_t)h * VD + v_base + v0, t)) = o;
      }
    }
    settle_chunk();
  }
  if (ht_out) {
    float* dst = ht_out + (size_t)bh * KD * VD;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * wv + 4 * lg + r, col = v_base + 16 * ct + lc;
        dst[vf ? col * KD + kr : kr * VD + col] = st[ct][r];
      }
  }
}

}  // namespace rewy
