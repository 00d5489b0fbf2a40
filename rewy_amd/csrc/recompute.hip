// Forward recomputation inside the backward (recompute policy).
//
// Replaces FLA's recompute_w_u_fwd and chunk_gated_delta_rule_fwd_h as called at
// reference backends/backward.py:110-118 (GDN / DeltaNet always; KDA / GDN2 when
// the forward did not save its intermediates), plus the intra-chunk scores of
// FLA's chunk_bwd_dv_local for the scalar-gate families.
//
//   fdr_prepare_wu (one work-group per chunk-head):
//     w   = Akk (b k 2^g)        bf16 [B,T,H,K]
//     u   = Akk (w_gate v)       bf16 [B,T,H,V]
//     qg  = q 2^g, kg = k 2^(g_last - g)           (vector gates, optional)
//     Aqk = scale tril(q k^T 2^(g_i - g_s))        (scalar / no gate, optional)
//   fdr_fwd_h (sequential over chunks, one work-group per (batch, head, value tile)):
//     h_c -> h[c] (bf16); v_new_c = u_c - w_c h_c (bf16); h_{c+1} = lambda_c h_c + kg_c^T v_new_c
//   fdr_fwd_h_wy: the two in one sweep (w, u formed one chunk ahead inside the scan);
//   fdr_fwd_h_u: the same sweep storing only h / v_new, with w read (or formed) and u and
//     a vector gate's kg formed (or kg read) -- the paired recurrences' scan
//
// The WY products are computed transposed (w^T = E^T A^T) so the accumulator
// layout stores w and u contiguously; A and E are split into bf16 hi + lo (16
// mantissa bits each; three MFMAs per product, the lo x lo term dropped).
#include "rewy_amd.h"

#include "scan_body.hpp"

namespace rewy {

namespace rec {
constexpr int LDT = 72;
constexpr int T128 = KD * LDT * 2;
}

// ------------------------------------------------------------------------------------------
// fdr_prepare_wu
// ------------------------------------------------------------------------------------------
template <int GATE, bool VEC_B, bool WANT_QKG, bool WANT_AQK, bool MAP, bool WANT_U = true>
__global__ __launch_bounds__(256) void prepare_wu_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, bf16* __restrict__ w_out,
    bf16* __restrict__ u_out, bf16* __restrict__ qg_out, bf16* __restrict__ kg_out,
    float* __restrict__ aqk_out, int T, int H, int HQ, float scale, const int* __restrict__ cu,
    const int* __restrict__ ci) {
  using rec::LDT;
  // Scalar or no gate with scalar beta: k is staged raw and E = (beta k) 2^g is formed
  // per operand fragment (one factor pair per token row), so Aqk reads k from LDS too
  // instead of re-fetching it from HBM.
  constexpr bool RAWK = GATE != RG_VECTOR && !VEC_B;
  // E = b k 2^g (or raw k) and Z = w_gate v rows [t][.] in bf16 (E rounded as FLA's
  // recompute_w_u_fwd rounds k beta 2^g before its dot), swizzled for transposed reads;
  // A rows hi/lo
  __shared__ __attribute__((aligned(16))) bf16 eH[C * KD];
  __shared__ __attribute__((aligned(16))) bf16 zH[C * VD];
  __shared__ __attribute__((aligned(16))) bf16 sAh[C][LDT];
  __shared__ __attribute__((aligned(16))) bf16 sAl[C][LDT];
  __shared__ float sG[C];
  __shared__ float sB[C];
  __shared__ __attribute__((aligned(16))) float sGe[C];   // RAWK: 2^g per row

  const int NT = T / C;
  const int blk = blockIdx.x;
  // heads run fastest: work-groups in flight together read neighbouring heads of
  // the same tokens, i.e. contiguous HBM rows
  const int h = blk % H;
  const int c = (blk / H) % NT;
  const int b = blk / (H * NT);
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int lc = l & 15, lg = l >> 4;
  const Rows<MAP> rw = chunk_rows<MAP>(cu, ci, b, c, T);
  const size_t tok0 = rw.tok0;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;
  const size_t kofs = tok0 * rsk + (size_t)h * KD;
  const size_t vofs = tok0 * rsv + (size_t)h * VD;
  const QKRows qr = qk_rows(tok0, h, H, HQ);   // raw q / k rows (grouped value heads: HQ < H)

  // Loads first, all in flight together: every row piece of E, Z and A with its rows' gate
  // and beta (below), the row gate and beta that later phases read from LDS, then Aqk's q
  // fragments (wave wv: row tile wv, used last).
  const int trow = tid & (C - 1);
  const float gv = (GATE == RG_SCALAR) ? g[(tok0 + rw.clamp(trow)) * H + h] : 0.f;
  const float bv = VEC_B ? 0.f : *rw.src(beta + (tok0 + trow) * H + h, trow);
  // ---- stage E = b k 2^g, Z = w_gate v (bf16) and A (hi/lo) row-major, coalesced 16-byte rows ----
  // Every row piece this thread stages is fetched first (1024 pieces of 8 columns: row p >> 4,
  // p = tid + 256 i), so the loads are in flight together instead of one round trip per piece.
  // The qg / kg pieces (vector gates) are the same rows and columns: k and g serve both.
  u32x4 rkx[4], rvx[4], rbx[4], rwx[4], rqx[4];
  f32x4 ra4[4], rg0[4], rg1[4];
  f32x4 rgl0, rgl1;
  float rgs[4], rbs[4];      // scalar gate and beta of each piece's row
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i;
    const int t = p >> 4, c0 = 8 * (p & 15);
    rgs[i] = (GATE == RG_SCALAR) ? g[(tok0 + rw.clamp(t)) * H + h] : 0.f;
    rbs[i] = VEC_B ? 0.f : *rw.src(beta + (tok0 + t) * H + h, t);
    rkx[i] = *reinterpret_cast<const u32x4*>(rw.src(k + qr.ofs + (size_t)t * qr.rs + c0, t));
    if constexpr (WANT_U) rvx[i] = *reinterpret_cast<const u32x4*>(rw.src(v + vofs + (size_t)t * rsv + c0, t));
    ra4[i] = *reinterpret_cast<const f32x4*>(tril_src(rw.src(akk + ((tok0 + t) * H + h) * C + 4 * (p & 15), t), t,
                                                      p & 15));
    if constexpr (GATE == RG_VECTOR) {
      rg0[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rw.clamp(t) * rsk + c0);
      rg1[i] = *reinterpret_cast<const f32x4*>(g + kofs + (size_t)rw.clamp(t) * rsk + c0 + 4);
    }
    if constexpr (VEC_B) {
      rbx[i] = *reinterpret_cast<const u32x4*>(rw.src(bgate + kofs + (size_t)t * rsk + c0, t));
      if constexpr (WANT_U) rwx[i] = *reinterpret_cast<const u32x4*>(rw.src(wgate + vofs + (size_t)t * rsv + c0, t));
    }
    if constexpr (WANT_QKG && GATE == RG_VECTOR)
      rqx[i] = *reinterpret_cast<const u32x4*>(rw.src(q + qr.ofs + (size_t)t * qr.rs + c0, t));
  }
  if constexpr (WANT_QKG && GATE == RG_VECTOR) {
    // g_last of this thread's 8 columns (the same for its four pieces)
    const float* gl = g + kofs + (size_t)rw.clamp(C - 1) * rsk + 8 * (tid & 15);
    rgl0 = *reinterpret_cast<const f32x4*>(gl);
    rgl1 = *reinterpret_cast<const f32x4*>(gl + 4);
  }
  bf16x8 qa[4];
  if constexpr (WANT_AQK) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qa[ks] = *reinterpret_cast<const bf16x8*>(
          rw.src(q + qr.ofs + (size_t)(16 * wv + lc) * qr.rs + 32 * ks + 8 * lg, 16 * wv + lc));
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i;
    const int t = p >> 4, ch = p & 15, c0 = 8 * ch;
    const bf16x8 kx = __builtin_bit_cast(bf16x8, rkx[i]);
    const bf16x8 vx = WANT_U ? __builtin_bit_cast(bf16x8, rvx[i]) : bf16x8{};
    float ge[8], be[8], we[8];
    if constexpr (GATE == RG_VECTOR) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ge[j] = fast_exp2(rg0[i][j]);
        ge[j + 4] = fast_exp2(rg1[i][j]);
      }
    } else {
      const float s0 = (GATE == RG_SCALAR) ? fast_exp2(rgs[i]) : 1.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ge[j] = s0;
    }
    if constexpr (VEC_B) {
      const bf16x8 bx = __builtin_bit_cast(bf16x8, rbx[i]);
      const bf16x8 wx = WANT_U ? __builtin_bit_cast(bf16x8, rwx[i]) : bf16x8{};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        be[j] = to_f32(bx[j]);
        we[j] = to_f32(wx[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) be[j] = we[j] = rbs[i];
    }
    bf16x8 eh, zh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      eh[j] = RAWK ? kx[j] : to_bf16(be[j] * to_f32(kx[j]) * ge[j]);
      zh[j] = to_bf16(we[j] * to_f32(vx[j]));
    }
    store_tr_chunk<16>(eH, t, ch, __builtin_bit_cast(u32x4, eh));
    if constexpr (WANT_U) store_tr_chunk<16>(zH, t, ch, __builtin_bit_cast(u32x4, zh));
    // A rows: 64 x 64 fp32 = 1024 pieces of 4, one per (i, thread) here
    bf16x4 alo;
    const bf16x4 ahi = split_hi4(tril_piece(ra4[i], t, ch), alo);
    *reinterpret_cast<bf16x4*>(&sAh[t][4 * ch]) = ahi;
    *reinterpret_cast<bf16x4*>(&sAl[t][4 * ch]) = alo;
    // qg = q 2^g, kg = k 2^(g_last - g) (vector gates): elementwise, coalesced
    if constexpr (WANT_QKG && GATE == RG_VECTOR) {
      const bf16x8 qx = __builtin_bit_cast(bf16x8, rqx[i]);
      bf16x8 oq, ok;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float gj = j < 4 ? rg0[i][j] : rg1[i][j - 4];
        const float glj = j < 4 ? rgl0[j] : rgl1[j - 4];
        oq[j] = to_bf16(to_f32(qx[j]) * fast_exp2(gj));
        ok[j] = to_bf16(to_f32(kx[j]) * fast_exp2(glj - gj));
      }
      *reinterpret_cast<bf16x8*>(rw.dst(qg_out + kofs + (size_t)t * rsk + c0, t)) = oq;
      *reinterpret_cast<bf16x8*>(rw.dst(kg_out + kofs + (size_t)t * rsk + c0, t)) = ok;
    }
  }
  if (tid < C) {
    sG[tid] = gv;
    sB[tid] = bv;
    sGe[tid] = (GATE == RG_SCALAR) ? fast_exp2(gv) : 1.f;
  }
  lds_barrier();

  // ---- w^T = E^T A^T, u^T = Z^T A^T: B operand = A rows (t), contiguous s, from LDS ----
  // wave wv: output rows (k or v) [32 wv, 32 wv + 32), all 64 token columns
  // (!WANT_U: w only; the forward scan that reads w forms u itself, fdr_fwd_h_u)
  {
#pragma unroll
    for (int which = 0; which < (WANT_U ? 2 : 1); ++which) {
      const bf16* srcH = which == 0 ? eH : zH;
      bf16* dst = which == 0 ? w_out + kofs : u_out + vofs;
      const size_t rs = which == 0 ? rsk : rsv;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int row0 = 32 * wv + 16 * rt;
        bf16x8 x0 = frag_tr<16>(srcH, 0, row0);    // E^T rows (k or v), over s
        bf16x8 x1 = frag_tr<16>(srcH, 32, row0);
        if (RAWK && which == 0) {
          // element e of the fragment is token row 8 (l >> 4) + e (+ 32)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t0 = 8 * lg + e, t1 = t0 + 32;
            x0[e] = to_bf16(sB[t0] * to_f32(x0[e]) * sGe[t0]);
            x1[e] = to_bf16(sB[t1] * to_f32(x1[e]) * sGe[t1]);
          }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          f32x4 acc = zero4();
          acc = mfma(x0, frag(&sAh[16 * tt][0], LDT), acc);
          acc = mfma(x0, frag(&sAl[16 * tt][0], LDT), acc);
          acc = mfma(x1, frag(&sAh[16 * tt][32], LDT), acc);
          acc = mfma(x1, frag(&sAl[16 * tt][32], LDT), acc);
          // lane: token t = 16 tt + lc, columns row0 + 4 lg .. +3
          bf16x4 o;
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = to_bf16(acc[r]);
          *reinterpret_cast<bf16x4*>(rw.dst(dst + (size_t)(16 * tt + lc) * rs + row0 + 4 * lg, 16 * tt + lc)) = o;
        }
      }
    }
  }

  // ---- Aqk = scale tril(q k^T 2^(g_i - g_s)) for the scalar / no-gate families ----
  if constexpr (WANT_AQK) {
    // wave wv: row tile I = wv, all four column tiles
    const int I = wv;
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      f32x4 acc = zero4();
      if (J <= I) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 a = qa[ks];
          bf16x8 bq;
          if constexpr (RAWK) bq = frag_row<16>(eH, 16 * J, 32 * ks);
          else
            bq = *reinterpret_cast<const bf16x8*>(
                rw.src(k + qr.ofs + (size_t)(16 * J + lc) * qr.rs + 32 * ks + 8 * lg, 16 * J + lc));
          acc = mfma(a, bq, acc);
        }
      }
      const int s = 16 * J + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        float f = (i >= s) ? scale : 0.f;
        if constexpr (GATE == RG_SCALAR) f = (i >= s) ? scale * fast_exp2(sG[i] - sG[s]) : 0.f;
        *rw.dst(aqk_out + ((tok0 + i) * H + h) * C + s, i) = acc[r] * f;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// fdr_fwd_h
// ------------------------------------------------------------------------------------------
template <int BV, int GATE>
struct FwdSmem {
  static constexpr int LDK = KD + 8;
  static constexpr int LDT = C + 8;
  // kg, h^T and lambda, which a step's tail reads (the update, the stores), per chunk parity,
  // so a step starts without a barrier
  bf16 w[C][LDK];          // w rows: A operand of w h           (contraction over K)
  bf16 k[2][C * KD];       // kg rows (swizzled): A operand of kg^T v_new (over T, transposed reads)
  bf16 hT[2][BV][LDK];     // h^T:    B operand of w h
  bf16 vT[BV][LDT];        // v_new^T: B operand of kg^T v_new
  bf16 u[C * BV];          // u rows [t][v] (swizzled): read transposed in the accumulator layout
  float lam[2][KD];
};

template <int BV, int GATE, bool MAP>
__global__ __launch_bounds__(512) void fwd_h_kernel(
    const bf16* __restrict__ k, const bf16* __restrict__ w, const bf16* __restrict__ u,
    const float* __restrict__ g, const float* __restrict__ h0, bf16* __restrict__ h_out,
    bf16* __restrict__ vnew_out, float* __restrict__ ht_out, int T, int H, const int* __restrict__ chunk_off,
    int vf, int HQ, const int* __restrict__ cu) {
  using S = FwdSmem<BV, GATE>;
  __shared__ S sm;
  constexpr int NVT = VD / BV;
  constexpr int NCT = BV / 16;
  constexpr int NTH = 512;
  const int logical = xcd_logical_block();
  const int vt = logical % NVT;
  const int bh = logical / NVT;
  const int b = bh / H, h = bh % H;
  // chunks [c0, c0 + NT) of the packed token axis: row b of T tokens, or sequence b of
  // a variable-length batch (chunk_off: cumulative chunk counts; clamped to the T / C
  // chunks there are, an empty sequence passes its state through)
  const int c0 = chunk_off ? min(max(chunk_off[b], 0), T / C) : b * (T / C);
  const int NT = chunk_off ? max(min(chunk_off[b + 1], T / C) - c0, 0) : T / C;
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int v_base = vt * BV;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;

  // state rows [16 wv, 16 wv + 16)
  f32x4 st[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    f32x4 a = zero4();
    if (h0) {
      const float* src = h0 + (size_t)bh * KD * VD;     // [K,V] or, state_v_first (vf), [V,K]
      const int col = v_base + 16 * ct + (l & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * wv + 4 * (l >> 4) + r;
        a[r] = src[vf ? col * KD + kr : kr * VD + col];
      }
    }
    st[ct] = a;
  }
  constexpr int DCT = NCT >= 2 ? NCT / 2 : 1;
  const int drow = wv & 3;
  const int dct0 = DCT * (wv >> 2);
  const bool has_dr = dct0 < NCT;

  u32x4 rw[2];
  u32x4 rk[2];
  // u rows: 16-byte pieces, every lane one or more (clamped, so the counts are static)
  constexpr int CHV = BV / 8;
  constexpr int NPU = C * CHV;
  constexpr int NU = (NPU + NTH - 1) / NTH;
  u32x4 ru[NU];
  float rg_last = 0.f, rg_tok[2] = {0.f, 0.f};   // scalar gate: last row, the 2 rows this thread stages
  auto load_chunk = [&](int c) {
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    const bf16* wb = w + tok0 * rsk + (size_t)h * KD;
    // gate first: its consumer (lambda) is the first thing staged.  Every lane
    // issues the same loads (clamped indices): no branch makes the vector-memory
    // wait counts lane- or wave-dependent.
    if constexpr (GATE == RG_VECTOR) {
      rg_last = g[((tok0 + rs_.clamp(C - 1)) * H + h) * KD + (tid & (KD - 1))];
    } else if constexpr (GATE == RG_SCALAR) {
#pragma unroll
      for (int i = 0; i < 2; ++i) rg_tok[i] = g[(tok0 + rs_.clamp((tid + NTH * i) >> 4)) * H + h];
      rg_last = g[(tok0 + rs_.clamp(C - 1)) * H + h];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      rw[i] = *reinterpret_cast<const u32x4*>(rs_.src(wb + (size_t)(p >> 4) * rsk + (p & 15) * 8, p >> 4));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      const QKRows kr_ = qk_rows(tok0, h, H, HQ);     // k: raw (HQ heads) for scalar gates, kg (HQ = H) else
      rk[i] = *reinterpret_cast<const u32x4*>(rs_.src(k + kr_.ofs + (size_t)(p >> 4) * kr_.rs + (p & 15) * 8, p >> 4));
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int p = min(tid + NTH * i, NPU - 1);
      ru[i] = *reinterpret_cast<const u32x4*>(
          rs_.src(u + (tok0 + p / CHV) * rsv + (size_t)h * VD + v_base + (p % CHV) * 8, p / CHV));
    }
  };
  auto stage_chunk = [&](int db) {
    if constexpr (GATE == RG_VECTOR) {
      if (tid < KD) sm.lam[db][tid] = fast_exp2(rg_last);
    } else if constexpr (GATE == RG_SCALAR) {
      if (tid < KD) sm.lam[db][tid] = fast_exp2(rg_last);
    } else {
      if (tid < KD) sm.lam[db][tid] = 1.f;
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int p = tid + NTH * i;
      if (NPU % NTH == 0 || p < NPU) store_tr_chunk<CHV>(sm.u, p / CHV, p % CHV, ru[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      *reinterpret_cast<u32x4*>(&sm.w[p >> 4][(p & 15) * 8]) = rw[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + NTH * i;
      u32x4 kq = rk[i];
      // scalar gate: kg = k 2^(g_last - g_t), the row's factor from registers
      if constexpr (GATE == RG_SCALAR) kq = scale_bf16x8(kq, fast_exp2(rg_last - rg_tok[i]));
      store_tr_chunk<16>(sm.k[db], p >> 4, p & 15, kq);
    }
  };

  auto settle_chunk = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      settle(rw[i]);
      settle(rk[i]);
    }
#pragma unroll
    for (int i = 0; i < NU; ++i) settle(ru[i]);
    settle(rg_last);
    settle(rg_tok[0]);
    settle(rg_tok[1]);
  };
  if (NT > 0) {
    load_chunk(0);
    settle_chunk();
  }
  for (int c = 0; c < NT; ++c) {
    // no barrier: w and u were last read before the previous step's last barrier, and kg,
    // h^T and lambda have a buffer per chunk parity
    const int db = c & 1;
    stage_chunk(db);
    load_chunk(c + 1 < NT ? c + 1 : c);    // (the last chunk re-fetches itself: no branch)
    const Rows<MAP> rs_ = seq_chunk_rows<MAP>(cu, b, c, c0 + c);
    const size_t tok0 = rs_.tok0;
    // h_c -> LDS (transposed, bf16); the same rounded values feed w h, as stored
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = to_bf16(st[ct][r]);
      *reinterpret_cast<bf16x4*>(&sm.hT[db][16 * ct + (l & 15)][16 * wv + 4 * (l >> 4)]) = v4;
    }
    lds_barrier();
    // v_new tiles = u - w h
    if (has_dr) {
#pragma unroll
      for (int cc = 0; cc < DCT; ++cc) {
        const int ct = dct0 + cc;
        // u rows 16 drow + 4 (l >> 4) .. + 3 of column 16 ct + (l & 15), transposed read
        const int lc = l & 15;
        const bf16x4 u4 = ds_read_tr4(sm.u + tr_off<CHV>(16 * drow + 4 * (l >> 4) + (lc >> 2), 16 * ct + 4 * (lc & 3)));
        f32x4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = -to_f32(u4[r]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          a = mfma(frag(&sm.w[16 * drow][32 * ks], S::LDK), frag(&sm.hT[db][16 * ct][32 * ks], S::LDK), a);
        bf16x4 v4;
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = to_bf16(-a[r]);
        *reinterpret_cast<bf16x4*>(&sm.vT[16 * ct + (l & 15)][16 * drow + 4 * (l >> 4)]) = v4;
      }
    }
    lds_barrier();
    // h <- lambda h + kg^T v_new
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) a[r] = st[ct][r] * sm.lam[db][16 * wv + 4 * (l >> 4) + r];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a = mfma(frag_tr<16>(sm.k[db], 32 * ks, 16 * wv), frag(&sm.vT[16 * ct][32 * ks], S::LDT), a);
      st[ct] = a;
    }
    // stores of h_c and v_new_c from the transposed LDS copies (lanes run over rows)
    {
      const size_t hb = ((size_t)(c0 + c) * H + h) * KD * VD;
      // Every lane issues the same number of stores (tasks beyond the tile are written
      // twice, with the same data): static vector-memory wait counts.
      // per wave task a block of 16 columns (h rows k / v_new rows t) by 32 value rows, 16-lane
      // group g taking 8 of them (two transposed reads per 16-byte piece)
      constexpr int RB = BV / 8, RQ = RB >= 4 ? RB / 4 : 1, NW = NTH / 64;
      constexpr int NTK = (KD / 16) * RQ, NTR = (C / 16) * RQ;
#pragma unroll
      for (int i = 0; i < (NTK + NW - 1) / NW; ++i) {
        const int tk = (wv + NW * i) % NTK;
        const int kr0 = 16 * (tk % (KD / 16)), v0 = 8 * ((4 * (tk / (KD / 16)) + (l >> 4)) % RB);
        const bf16x8 o = col8_tr(&sm.hT[db][0][0], S::LDK, v0, kr0, l);
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
    settle_chunk();    // the next chunk's operands, settled behind this chunk's stores
  }
  if (ht_out) {
    float* dst = ht_out + (size_t)bh * KD * VD;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * wv + 4 * (l >> 4) + r, col = v_base + 16 * ct + (l & 15);
        dst[vf ? col * KD + kr : kr * VD + col] = st[ct][r];
      }
  }
}

// fdr_fwd_h_wy / fdr_fwd_h_u: the scan body (scan_body.hpp) as a kernel of its own
template <int BV, int GATE, bool VEC_B, bool MAP, bool WG = false, bool NOST = false, bool KGIN = false>
__global__ __launch_bounds__(512) void fwd_h_wy_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const float* __restrict__ h0,
    bf16* __restrict__ w_out, bf16* __restrict__ qg_out, bf16* __restrict__ kg_out, bf16* __restrict__ h_out,
    bf16* __restrict__ vnew_out, float* __restrict__ ht_out, int T, int H, const int* __restrict__ chunk_off,
    int vf, int HQ, const int* __restrict__ cu, const bf16* __restrict__ w_in = nullptr) {
  __shared__ FwdWySmem<BV> sm;
  fwd_h_wy_body<BV, GATE, VEC_B, MAP, WG, NOST, KGIN>(sm, xcd_logical_block(), q, k, v, g, beta, bgate, wgate, akk,
                                                      h0, w_out, qg_out, kg_out, h_out, vnew_out, ht_out, T, H,
                                                      chunk_off, vf, HQ, cu, w_in);
}

template <int BV, int GATE, bool VEC_B, bool WG = false, bool NOST = false, bool KGIN = false>
static hipError_t launch_fwd_h_wy(const void* q, const void* k, const void* v, const float* g, const float* beta,
                                  const void* bg, const void* wg, const float* akk, const float* h0, void* w,
                                  void* qg, void* kg, void* h, void* vnew, float* ht, int B, int T, int H,
                                  hipStream_t s, const int* co, int vf, int HQ, const int* cu,
                                  const void* w_in = nullptr) {
#define FW_LAUNCH(MAP)                                                                                             \
  hipLaunchKernelGGL((fwd_h_wy_kernel<BV, GATE, VEC_B, MAP, WG, NOST, KGIN>), dim3(B * H * (VD / BV)), dim3(512), 0, \
                     s,                                                                                           \
                     (const bf16*)q, (const bf16*)k, (const bf16*)v, g, beta, (const bf16*)bg, (const bf16*)wg, akk, \
                     h0, (bf16*)w, (bf16*)qg, (bf16*)kg, (bf16*)h, (bf16*)vnew, ht, T, H, co, vf, HQ, cu,        \
                     (const bf16*)w_in)
  if (cu) FW_LAUNCH(true);
  else FW_LAUNCH(false);
#undef FW_LAUNCH
  return hipGetLastError();
}

template <int GATE, bool VEC_B, bool QKG, bool AQK, bool WU = true>
static hipError_t launch_prepare(const void* q, const void* k, const void* v, const float* g,
                                 const float* beta, const void* bg, const void* wg, const float* akk,
                                 void* w, void* u, void* qg, void* kg, float* aqk, int B, int T, int H, int HQ,
                                 float scale, hipStream_t s, const int* cu, const int* ci) {
#define P_LAUNCH(MAP)                                                                                            \
  hipLaunchKernelGGL((prepare_wu_kernel<GATE, VEC_B, QKG, AQK, MAP, WU>), dim3(B * H * (T / C)), dim3(256), 0, s, \
                     (const bf16*)q, (const bf16*)k, (const bf16*)v, g, beta, (const bf16*)bg, (const bf16*)wg, \
                     akk, (bf16*)w, (bf16*)u, (bf16*)qg, (bf16*)kg, aqk, T, H, HQ, scale, cu, ci)
  if (cu) P_LAUNCH(true);
  else P_LAUNCH(false);
#undef P_LAUNCH
  return hipGetLastError();
}

template <int BV, int GATE>
static hipError_t launch_fwd_h(const void* k, const void* w, const void* u, const float* g, const float* h0,
                               void* h, void* vnew, float* ht, int B, int T, int H, hipStream_t s,
                               const int* co, int vf, int HQ, const int* cu) {
#define F_LAUNCH(MAP)                                                                                            \
  hipLaunchKernelGGL((fwd_h_kernel<BV, GATE, MAP>), dim3(B * H * (VD / BV)), dim3(512), 0, s, (const bf16*)k,     \
                     (const bf16*)w, (const bf16*)u, g, h0, (bf16*)h, (bf16*)vnew, ht, T, H, co, vf, HQ, cu)
  if (cu) F_LAUNCH(true);
  else F_LAUNCH(false);
#undef F_LAUNCH
  return hipGetLastError();
}

}  // namespace rewy

using namespace rewy;

// B rows of T tokens, or (cu, ci) a packed batch of T / 64 chunks
static hipError_t prepare_dispatch(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                   const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                                   void* w, void* u, void* qg, void* kg, float* Aqk, int B, int T, int H,
                                   int qk_heads, float scale, hipStream_t stream, const int* cu, const int* ci) {
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ || (b_gate && HQ != H)) return hipErrorInvalidValue;
  if (!k || !Akk || !w) return hipErrorInvalidValue;
  const bool vec_b = b_gate != nullptr;
  if (vec_b && (!w_gate || gate_mode != RG_VECTOR)) return hipErrorInvalidValue;
  if (!vec_b && !beta) return hipErrorInvalidValue;
  if (gate_mode != RG_NONE && !g) return hipErrorInvalidValue;
  const bool want_qkg = qg != nullptr || kg != nullptr;
  if (want_qkg && (!qg || !kg || !q || gate_mode != RG_VECTOR)) return hipErrorInvalidValue;
  const bool want_aqk = Aqk != nullptr;
  if (want_aqk && (!q || gate_mode == RG_VECTOR)) return hipErrorInvalidValue;
#define P_ARGS q, k, v, g, beta, b_gate, w_gate, Akk, w, u, qg, kg, Aqk, B, T, H, HQ, scale, stream, cu, ci
  if (!u) {
    // w (and, vector gates, optionally qg, kg; scalar / no gate, optionally Aqk) only, for the
    // forward scan that forms u itself (fdr_fwd_h_u)
    switch (gate_mode) {
      case RG_NONE:
        return want_aqk ? launch_prepare<RG_NONE, false, false, true, false>(P_ARGS)
                        : launch_prepare<RG_NONE, false, false, false, false>(P_ARGS);
      case RG_SCALAR:
        return want_aqk ? launch_prepare<RG_SCALAR, false, false, true, false>(P_ARGS)
                        : launch_prepare<RG_SCALAR, false, false, false, false>(P_ARGS);
      case RG_VECTOR:
        if (vec_b)
          return want_qkg ? launch_prepare<RG_VECTOR, true, true, false, false>(P_ARGS)
                          : launch_prepare<RG_VECTOR, true, false, false, false>(P_ARGS);
        return want_qkg ? launch_prepare<RG_VECTOR, false, true, false, false>(P_ARGS)
                        : launch_prepare<RG_VECTOR, false, false, false, false>(P_ARGS);
      default: return hipErrorInvalidValue;
    }
  }
  if (!v) return hipErrorInvalidValue;
  switch (gate_mode) {
    case RG_NONE:
      return want_aqk ? launch_prepare<RG_NONE, false, false, true>(P_ARGS)
                      : launch_prepare<RG_NONE, false, false, false>(P_ARGS);
    case RG_SCALAR:
      return want_aqk ? launch_prepare<RG_SCALAR, false, false, true>(P_ARGS)
                      : launch_prepare<RG_SCALAR, false, false, false>(P_ARGS);
    case RG_VECTOR:
      if (vec_b)
        return want_qkg ? launch_prepare<RG_VECTOR, true, true, false>(P_ARGS)
                        : launch_prepare<RG_VECTOR, true, false, false>(P_ARGS);
      return want_qkg ? launch_prepare<RG_VECTOR, false, true, false>(P_ARGS)
                      : launch_prepare<RG_VECTOR, false, false, false>(P_ARGS);
    default:
      return hipErrorInvalidValue;
  }
#undef P_ARGS
}

extern "C" hipError_t fdr_prepare_wu(const void* q, const void* k, const void* v, const float* g,
                                     int gate_mode, const float* beta, const void* b_gate,
                                     const void* w_gate, const float* Akk, void* w, void* u, void* qg,
                                     void* kg, float* Aqk, int B, int T, int H, int qk_heads, int K, int V,
                                     int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  return prepare_dispatch(q, k, v, g, gate_mode, beta, b_gate, w_gate, Akk, w, u, qg, kg, Aqk, B, T, H, qk_heads,
                          scale, stream, nullptr, nullptr);
}

extern "C" hipError_t fdr_prepare_wu_varlen(const void* q, const void* k, const void* v, const float* g,
                                            int gate_mode, const float* beta, const void* b_gate,
                                            const void* w_gate, const float* Akk, void* w, void* u, void* qg,
                                            void* kg, float* Aqk, const int* cu_seqlens, const int* chunk_indices,
                                            int num_chunks, int H, int qk_heads, int K, int V, int chunk,
                                            float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || num_chunks <= 0 || H <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return prepare_dispatch(q, k, v, g, gate_mode, beta, b_gate, w_gate, Akk, w, u, qg, kg, Aqk, 1, num_chunks * C, H,
                          qk_heads, scale, stream, cu_seqlens, chunk_indices);
}

// Value-tile width of the forward scans: as the state recurrence's (the narrowest tile with at
// most 256 work-groups, 64 beyond); measured alike for fdr_fwd_h and fdr_fwd_h_wy (B*H = 96,
// T = 4096: fwd_h_wy 327 us at 64-wide vs 524 at 32-wide; B*H = 48: 266 at 32-wide vs 446 at 16).
static int fwd_default_bv(int B, int H) {
  const int bh = B * H;
  if (bh * 8 <= 256) return 16;
  if (bh * 4 <= 256) return 32;
  return 64;
}

// B rows of T tokens, or (co) B sequences packed along T tokens on 64-token boundaries,
// or (co, cu) B sequences packed anywhere along the token axis, in T / 64 chunks
static hipError_t fwd_h_dispatch(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                                 const float* h0, void* h, void* v_new, float* ht, int B, int T, int H, int HQ,
                                 int K, int V, int chunk, int value_block, hipStream_t stream, const int* co,
                                 int vf, const int* cu) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (HQ <= 0) HQ = H;
  if (H % HQ) return hipErrorInvalidValue;
  if (!k || !w || !u || !h || !v_new) return hipErrorInvalidValue;
  if (gate_mode != RG_NONE && !g) return hipErrorInvalidValue;
  if (cu && !co) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : fwd_default_bv(B, H);
#define F_ARGS k, w, u, g, h0, h, v_new, ht, B, T, H, stream, co, vf, HQ, cu
#define F_BV(G)                                                     \
  switch (bv) {                                                     \
    case 16: return launch_fwd_h<16, G>(F_ARGS);                    \
    case 32: return launch_fwd_h<32, G>(F_ARGS);                    \
    case 64: return launch_fwd_h<64, G>(F_ARGS);                    \
    default: return hipErrorInvalidValue;                           \
  }
  switch (gate_mode) {
    case RG_NONE: F_BV(RG_NONE)
    case RG_SCALAR: F_BV(RG_SCALAR)
    case RG_VECTOR: F_BV(RG_VECTOR)
    default: return hipErrorInvalidValue;
  }
#undef F_BV
#undef F_ARGS
}

extern "C" hipError_t fdr_fwd_h(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                                const float* h0, void* h, void* v_new, float* ht, int state_v_first, int B, int T,
                                int H, int k_heads, int K, int V, int chunk, int value_block, hipStream_t stream) {
  return fwd_h_dispatch(k, w, u, g, gate_mode, h0, h, v_new, ht, B, T, H, k_heads, K, V, chunk, value_block, stream,
                        nullptr, state_v_first ? 1 : 0, nullptr);
}

extern "C" hipError_t fdr_fwd_h_varlen(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                                       const float* h0, void* h, void* v_new, float* ht, int state_v_first,
                                       const int* chunk_offsets, const int* cu_seqlens, int N, int num_chunks,
                                       int H, int k_heads, int K, int V, int chunk, int value_block,
                                       hipStream_t stream) {
  if (!chunk_offsets || num_chunks <= 0) return hipErrorInvalidValue;
  return fwd_h_dispatch(k, w, u, g, gate_mode, h0, h, v_new, ht, N, num_chunks * C, H, k_heads, K, V, chunk,
                        value_block, stream, chunk_offsets, state_v_first ? 1 : 0, cu_seqlens);
}

// B rows of T tokens, or (co[, cu]) B sequences packed along T tokens as for fwd_h_dispatch
static hipError_t fwd_h_wy_dispatch(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                    const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                                    const float* h0, void* w, void* qg, void* kg, void* h, void* v_new, float* ht,
                                    int B, int T, int H, int HQ, int K, int V, int chunk, int value_block,
                                    hipStream_t stream, const int* co, int vf, const int* cu) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (HQ <= 0) HQ = H;
  if (H % HQ) return hipErrorInvalidValue;
  if (!k || !v || !Akk || !w || !h || !v_new) return hipErrorInvalidValue;
  const bool vec_b = b_gate != nullptr;
  if (vec_b && (!w_gate || gate_mode != RG_VECTOR || HQ != H)) return hipErrorInvalidValue;
  if (!vec_b && !beta) return hipErrorInvalidValue;
  if (gate_mode != RG_NONE && !g) return hipErrorInvalidValue;
  if (gate_mode == RG_VECTOR && (!q || !qg || !kg)) return hipErrorInvalidValue;
  if (cu && !co) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : fwd_default_bv(B, H);
#define FW_ARGS q, k, v, g, beta, b_gate, w_gate, Akk, h0, w, qg, kg, h, v_new, ht, B, T, H, stream, co, vf, HQ, cu
#define FW_BV(G, VB)                                                \
  switch (bv) {                                                     \
    case 16: return launch_fwd_h_wy<16, G, VB>(FW_ARGS);            \
    case 32: return launch_fwd_h_wy<32, G, VB>(FW_ARGS);            \
    case 64: return launch_fwd_h_wy<64, G, VB>(FW_ARGS);            \
    default: return hipErrorInvalidValue;                           \
  }
  switch (gate_mode) {
    case RG_NONE: FW_BV(RG_NONE, false)
    case RG_SCALAR: FW_BV(RG_SCALAR, false)
    case RG_VECTOR:
      if (vec_b) FW_BV(RG_VECTOR, true)
      FW_BV(RG_VECTOR, false)
    default: return hipErrorInvalidValue;
  }
#undef FW_BV
#undef FW_ARGS
}

extern "C" hipError_t fdr_fwd_h_wy(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                   const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                                   const float* h0, void* w, void* qg, void* kg, void* h, void* v_new, float* ht,
                                   int state_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk,
                                   int value_block, hipStream_t stream) {
  return fwd_h_wy_dispatch(q, k, v, g, gate_mode, beta, b_gate, w_gate, Akk, h0, w, qg, kg, h, v_new, ht, B, T, H,
                           qk_heads, K, V, chunk, value_block, stream, nullptr, state_v_first ? 1 : 0, nullptr);
}

// The forward scan with u formed in-kernel from v (and beta or w_gate) and Akk, w given:
// B rows of T tokens, or (co[, cu]) packed sequences as for fwd_h_dispatch
static hipError_t fwd_h_u_dispatch(const void* k, const void* kg, const void* w, const void* v, const float* g,
                                   int gate_mode, const float* beta, const void* b_gate, const void* w_gate,
                                   const float* Akk, const float* h0, void* h, void* v_new, float* ht, int B, int T,
                                   int H, int HQ, int K, int V, int chunk, int value_block, hipStream_t stream,
                                   const int* co, int vf, const int* cu) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  if (HQ <= 0) HQ = H;
  if (H % HQ) return hipErrorInvalidValue;
  if (kg && (gate_mode != RG_VECTOR || !w)) return hipErrorInvalidValue;   // kg read: vector gate, w given
  if (kg) {
    k = kg;            // one row per value head
    HQ = H;
  }
  if (!k || !v || !Akk || !h || !v_new) return hipErrorInvalidValue;
  const bool vec_b = w_gate != nullptr;
  if (vec_b && gate_mode != RG_VECTOR) return hipErrorInvalidValue;
  if (!vec_b && !beta) return hipErrorInvalidValue;
  if (!w && vec_b && (!b_gate || HQ != H)) return hipErrorInvalidValue;   // E = (b k) 2^g needs b
  if (gate_mode != RG_NONE && !g) return hipErrorInvalidValue;
  if (cu && !co) return hipErrorInvalidValue;
  const int bv = value_block > 0 ? value_block : fwd_default_bv(B, H);
  // w given: b_gate is not read (only u's Z = w_gate v; a non-null pointer selects VEC_B);
  // w NULL: w formed too (NOST), from b_gate (GDN2) or beta
#define FU_ARGS nullptr, k, v, g, beta, w ? w_gate : b_gate, w_gate, Akk, h0, nullptr, nullptr, nullptr, h, v_new, ht, \
                B, T, H, stream, co, vf, HQ, cu, w
#define FU_BV(G, VB)                                                                          \
  switch (bv) {                                                                               \
    case 16: return w ? launch_fwd_h_wy<16, G, VB, true>(FU_ARGS)                             \
                      : launch_fwd_h_wy<16, G, VB, false, true>(FU_ARGS);                     \
    case 32: return w ? launch_fwd_h_wy<32, G, VB, true>(FU_ARGS)                             \
                      : launch_fwd_h_wy<32, G, VB, false, true>(FU_ARGS);                     \
    case 64: return w ? launch_fwd_h_wy<64, G, VB, true>(FU_ARGS)                             \
                      : launch_fwd_h_wy<64, G, VB, false, true>(FU_ARGS);                     \
    default: return hipErrorInvalidValue;                                                     \
  }
#define FU_KG(VB)                                                                             \
  switch (bv) {                                                                               \
    case 16: return launch_fwd_h_wy<16, RG_VECTOR, VB, true, false, true>(FU_ARGS);          \
    case 32: return launch_fwd_h_wy<32, RG_VECTOR, VB, true, false, true>(FU_ARGS);          \
    case 64: return launch_fwd_h_wy<64, RG_VECTOR, VB, true, false, true>(FU_ARGS);          \
    default: return hipErrorInvalidValue;                                                     \
  }
  if (kg) {
    if (vec_b) FU_KG(true)
    FU_KG(false)
  }
  switch (gate_mode) {
    case RG_NONE: FU_BV(RG_NONE, false)
    case RG_SCALAR: FU_BV(RG_SCALAR, false)
    case RG_VECTOR:
      if (vec_b) FU_BV(RG_VECTOR, true)
      FU_BV(RG_VECTOR, false)
    default: return hipErrorInvalidValue;
  }
#undef FU_KG
#undef FU_BV
#undef FU_ARGS
}

extern "C" hipError_t fdr_fwd_h_u(const void* k, const void* kg, const void* w, const void* v, const float* g,
                                  int gate_mode, const float* beta, const void* b_gate, const void* w_gate,
                                  const float* Akk, const float* h0, void* h, void* v_new, float* ht, int state_v_first,
                                  int B, int T, int H, int k_heads, int K, int V, int chunk, int value_block,
                                  hipStream_t stream) {
  return fwd_h_u_dispatch(k, kg, w, v, g, gate_mode, beta, b_gate, w_gate, Akk, h0, h, v_new, ht, B, T, H, k_heads,
                          K, V, chunk, value_block, stream, nullptr, state_v_first ? 1 : 0, nullptr);
}

extern "C" hipError_t fdr_fwd_h_wy_varlen(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                          const float* beta, const void* b_gate, const void* w_gate,
                                          const float* Akk, const float* h0, void* w, void* qg, void* kg, void* h,
                                          void* v_new, float* ht, int state_v_first, const int* chunk_offsets,
                                          const int* cu_seqlens, int N, int num_chunks, int H, int qk_heads, int K,
                                          int V, int chunk, int value_block, hipStream_t stream) {
  if (!chunk_offsets || num_chunks <= 0) return hipErrorInvalidValue;
  return fwd_h_wy_dispatch(q, k, v, g, gate_mode, beta, b_gate, w_gate, Akk, h0, w, qg, kg, h, v_new, ht, N,
                           num_chunks * C, H, qk_heads, K, V, chunk, value_block, stream, chunk_offsets,
                           state_v_first ? 1 : 0, cu_seqlens);
}
