// Affine-step form of the two inter-chunk state recurrences, for launches whose
// batch x head count leaves most of the chip idle (the sequential chain then
// sets the time, not HBM).
//
// Both recurrences are affine in the state S (128 x V, fp32) once the chunk's
// operands are fixed:
//
//   backward (chunk c = NT-1 .. 0, FLA chunk_gated_delta_rule_bwd_dhu, reference
//   kernels/vector_state_gpu.py:28-43):
//     dR_c = kg_c dh + dv_c ;  dh <- diag(lam_c) dh + scale qg_c^T dO_c - w_c^T dR_c
//          = diag(lam_c) dh - M_c dh + Y_c,   M_c = w_c^T kg_c,  Y_c = scale qg_c^T dO_c - w_c^T dv_c
//   forward (chunk c = 0 .. NT-1, FLA chunk_gated_delta_rule_fwd_h):
//     v_new_c = u_c - w_c h ;  h <- diag(lam_c) h + kg_c^T v_new_c
//          = diag(lam_c) h - N_c h + Z_c,     N_c = kg_c^T w_c,  Z_c = kg_c^T u_c
//
// M_c / N_c (128 x 128) and Y_c / Z_c (128 x V) do not depend on the state, so
// they are formed for every chunk in parallel (affine_prep_kernel).  What stays
// sequential is one 128 x 128 by 128 x V product per chunk (affine_scan_kernel:
// one barrier per chunk, the step operands prefetched several chunks ahead in
// registers), and the per-chunk side outputs dR_c / v_new_c, which need the
// state, are again chunk-parallel (affine_side_kernel).  The state still enters
// the product as bf16 and the step matrix is rounded to bf16 once, the same
// error class as the direct form's bf16 dR / v_new operand.
//
// Layouts private to this file, per chunk-head (b, c, h), chunk-heads ordered
// (b, c, h) like the per-chunk states:
//   step matrix, bf16 "A-fragment order": 32 blocks (rt * 4 + ks) of 64 lanes x 8:
//     lane l of block (rt, ks) holds A[16 rt + (l & 15)][32 ks + 8 (l >> 4) + e], e = 0..7
//   offset, fp32 "accumulator order": 64 blocks (ct * 8 + rt) of 64 lanes x 4:
//     lane l of block (ct, rt) holds Y[16 rt + 4 (l >> 4) + r][16 ct + (l & 15)], r = 0..3
// so every scan load is one contiguous 1 KiB wave access straight into MFMA
// operand / accumulator registers.
#include "common.hpp"

#include "rewy_amd.h"

namespace rewy {

enum AffGate { AG_NONE = 0, AG_SCALAR = 1, AG_VECTOR = 2 };

constexpr int A_FRAG = KD * KD;   // bf16 elements of one chunk-head's step matrix
constexpr int Y_FRAG = KD * VD;   // fp32 elements of one chunk-head's offset

// ---------------------------------------------------------------------------
// prep: step matrix and offset of every chunk-head
// ---------------------------------------------------------------------------
// 80 KiB, two work-groups per CU: the K x K product's staging reuses the inputs'
// bytes after the last MFMA, and (backward with Aqk) kg is written over Aqk's bf16 tile
// once dv_local is formed.
struct PrepSmem {
  union {
    struct {
      bf16 xa[C * KD];     // A side of the K x K product, swizzled rows [t][k]: w (bwd) | kg (fwd)
      bf16 xq[C * KD];     // bwd: qg
      bf16 y0[C * VD];     // bwd: dO | fwd: u   (swizzled rows [t][v])
      bf16 dv[C * VD];     // bwd: dv_local, bf16 (swizzled rows)
    } in;
    bf16 m[KD][KD + 8];    // the K x K product, row-major, for the fragment-order store
  } t;
  union {
    struct {
      bf16 ah[C * C];      // bwd: Aqk (bf16), rows [t][s] (8-chunk swizzle)
    } a;
    bf16 xb[C * KD];       // B side of the K x K product: kg (bwd) | w (fwd)
  } s;
};

struct PrepArgs {
  const bf16* q;        // bwd: qg | q
  const bf16* k;        // kg | k
  const bf16* w;
  const float* g;
  const bf16* y_src;    // bwd: dO | fwd: u
  const float* aqk;     // bwd: Aqk, or null with dv_in
  const bf16* dv_in;
  bf16* a_frag;
  float* y_frag;
  bf16* dv_out;         // bwd with Aqk: dv_local out
  float scale;
};

// One chunk-head ch (in (b, c, h) order).
//   BWD: M = w^T kg, Y = scale qg^T dO - w^T dv  (dv = Aqk^T dO, or given)
//   FWD: N = kg^T w, Z = kg^T u
template <bool BWD, int GATE, bool DV_FROM_AQK>
__device__ __forceinline__ void prep_body(PrepSmem& sm, const PrepArgs& pa, int ch, int T, int H) {
  const bf16* __restrict__ q = pa.q;
  const bf16* __restrict__ k = pa.k;
  const bf16* __restrict__ w = pa.w;
  const float* __restrict__ g = pa.g;
  const bf16* __restrict__ y_src = pa.y_src;
  const float* __restrict__ aqk = pa.aqk;
  const bf16* __restrict__ dv_in = pa.dv_in;
  bf16* __restrict__ a_frag = pa.a_frag;
  float* __restrict__ y_frag = pa.y_frag;
  bf16* __restrict__ dv_out = pa.dv_out;
  const float scale = pa.scale;
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int NT = T / C;
  const int h = ch % H, c = (ch / H) % NT, b = ch / (H * NT);
  const size_t tok0 = (size_t)b * T + (size_t)c * C;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;
  const size_t kofs = tok0 * rsk + (size_t)h * KD, vofs = tok0 * rsv + (size_t)h * VD;

  // ---- stage: 1024 16-byte pieces per [64][128] tile, 2 per thread ----
  constexpr bool KG_LATE = BWD && DV_FROM_AQK;   // kg waits in registers for Aqk's LDS
  u32x4 kreg[2];
  float glast = 0.f;
  if constexpr (GATE == AG_SCALAR) glast = g[(tok0 + C - 1) * H + h];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, cc = p & 15;
    const size_t o = kofs + (size_t)t * rsk + cc * 8;
    u32x4 kk = *reinterpret_cast<const u32x4*>(k + o);
    const u32x4 ww = *reinterpret_cast<const u32x4*>(w + o);
    float gt = 0.f;
    if constexpr (GATE == AG_SCALAR) {
      gt = g[(tok0 + t) * H + h];
      kk = scale_bf16x8(kk, fast_exp2(glast - gt));      // kg = k 2^(g_last - g_t)
    }
    if constexpr (BWD) {
      store_tr_chunk<16>(sm.t.in.xa, t, cc, ww);
      if constexpr (KG_LATE) kreg[i] = kk;
      else store_tr_chunk<16>(sm.s.xb, t, cc, kk);
      u32x4 qq = *reinterpret_cast<const u32x4*>(q + o);
      if constexpr (GATE == AG_SCALAR) qq = scale_bf16x8(qq, fast_exp2(gt));   // qg = q 2^(g_t)
      store_tr_chunk<16>(sm.t.in.xq, t, cc, qq);
      if constexpr (DV_FROM_AQK) {
        // Aqk as one bf16, the precision of the reference's dv_local (FLA's dAv rounds A to
        // the dO dtype before its dot: kernels/kda_residual_npu_onchip.py:114-116)
        const f32x4 a = *reinterpret_cast<const f32x4*>(tril_src(aqk + ((tok0 + t) * H + h) * C + cc * 4, t, cc));
        bf16x4 hi;
#pragma unroll
        for (int r = 0; r < 4; ++r) hi[r] = to_bf16(tril_elem(a[r], t, 4 * cc + r));
        *reinterpret_cast<bf16x4*>(sm.s.a.ah + tr_off<8>(t, cc * 4)) = hi;
      } else {
        store_tr_chunk<16>(sm.t.in.dv, t, cc, *reinterpret_cast<const u32x4*>(dv_in + vofs + (size_t)t * rsv + cc * 8));
      }
    } else {
      store_tr_chunk<16>(sm.t.in.xa, t, cc, kk);
      store_tr_chunk<16>(sm.s.xb, t, cc, ww);
    }
    store_tr_chunk<16>(sm.t.in.y0, t, cc, *reinterpret_cast<const u32x4*>(y_src + vofs + (size_t)t * rsv + cc * 8));
  }
  lds_barrier();

  if constexpr (BWD && DV_FROM_AQK) {
    // dv[s][v] = sum_t Aqk[t][s] dO[t][v]: wave (rt = wv & 3) x column tiles 4 (wv >> 2) .. + 3
    const int rt = wv & 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ct = 4 * (wv >> 2) + j;
      f32x4 a = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 bo = frag_tr<16>(sm.t.in.y0, 32 * ks, 16 * ct);
        a = mfma(frag_tr<8>(sm.s.a.ah, 32 * ks, 16 * rt), bo, a);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sm.t.in.dv[tr_off<16>(16 * rt + 4 * (l >> 4) + r, 16 * ct + (l & 15))] = to_bf16(a[r]);
    }
    lds_barrier();                               // dv complete, Aqk dead
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;
      const int t = p >> 4, cc = p & 15;
      store_tr_chunk<16>(sm.s.xb, t, cc, kreg[i]);
      *reinterpret_cast<u32x4*>(dv_out + vofs + (size_t)t * rsv + cc * 8) =
          *reinterpret_cast<const u32x4*>(sm.t.in.dv + tr_off<16>(t, cc * 8));
    }
    lds_barrier();
  }

  // ---- K x K product and offset: wave wv owns output rows [16 wv, 16 wv + 16) ----
  const int rt = wv;
  bf16x8 af[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) af[ks] = frag_tr<16>(sm.t.in.xa, 32 * ks, 16 * rt);
  f32x4 pm[8];
  float* ydst = y_frag + (size_t)ch * Y_FRAG;
#pragma unroll
  for (int ct = 0; ct < 8; ++ct) {
    f32x4 a = zero4(), y = zero4();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      a = mfma(af[ks], frag_tr<16>(sm.s.xb, 32 * ks, 16 * ct), a);
      if constexpr (BWD) {
        y = mfma(af[ks], frag_tr<16>(sm.t.in.dv, 32 * ks, 16 * ct), y);     // w^T dv
      } else {
        y = mfma(af[ks], frag_tr<16>(sm.t.in.y0, 32 * ks, 16 * ct), y);     // kg^T u
      }
    }
    if constexpr (BWD) {
      f32x4 x = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        x = mfma(frag_tr<16>(sm.t.in.xq, 32 * ks, 16 * rt), frag_tr<16>(sm.t.in.y0, 32 * ks, 16 * ct), x);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = scale * x[r] - y[r];
    }
    pm[ct] = a;
    *reinterpret_cast<f32x4*>(ydst + ((ct * 8 + rt) * 64 + l) * 4) = y;
  }
  lds_barrier();                                  // every wave done with the staged inputs
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.t.m[16 * rt + 4 * (l >> 4) + r][16 * ct + (l & 15)] = to_bf16(pm[ct][r]);
  lds_barrier();
  bf16* adst = a_frag + (size_t)ch * A_FRAG;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 512 * i;                  // block p >> 6 = rt' * 4 + ks, lane p & 63
    const int blk = p >> 6, L = p & 63;
    const int row = 16 * (blk >> 2) + (L & 15), col = 32 * (blk & 3) + 8 * (L >> 4);
    *reinterpret_cast<u32x4*>(adst + (size_t)p * 8) = *reinterpret_cast<const u32x4*>(&sm.t.m[row][col]);
  }
}

template <bool BWD, int GATE, bool DV_FROM_AQK>
__global__ __launch_bounds__(512) void affine_prep_kernel(PrepArgs a, int T, int H) {
  __shared__ PrepSmem sm;
  prep_body<BWD, GATE, DV_FROM_AQK>(sm, a, blockIdx.x, T, H);
}

// forward and backward preparation in one launch: blocks [0, n) backward, [n, 2n) forward
template <int GATE, bool DV_FROM_AQK>
__global__ __launch_bounds__(512) void affine_prep_pair_kernel(PrepArgs bwd, PrepArgs fwd, int n, int T, int H) {
  __shared__ PrepSmem sm;
  if ((int)blockIdx.x < n) prep_body<true, GATE, DV_FROM_AQK>(sm, bwd, blockIdx.x, T, H);
  else prep_body<false, GATE, false>(sm, fwd, blockIdx.x - n, T, H);
}

// ---------------------------------------------------------------------------
// scan: S <- diag(lam_c) S - A_c S + Y_c, storing S before each step
// ---------------------------------------------------------------------------
struct ScanArgs {
  const bf16* a;
  const float* y;
  const float* g;
  const float* s0;
  bf16* s_out;
  float* s_final;
  int reverse;
  int vf;            // s0 / s_final in [V,K] (state_v_first) instead of [K,V]
};

// GATE is a template parameter so that the gate load is branch-free: a branch
// around a load makes the compiler's wait counts path-dependent, and it then
// waits for every outstanding load (the whole prefetch) at the join.
// NW waves, each owning RT = 8 / NW row tiles of 16 state rows (wave w: tiles w, w + NW, ...).
// Every wave reads the whole bf16 state from LDS per chunk; fewer waves read less but each
// runs a longer chain per chunk, and 8 measured fastest.
template <int NCT, int D, int GATE, int NW>
__global__ __launch_bounds__(64 * NW) void affine_scan_kernel(ScanArgs p0, ScanArgs p1, int nb0, int T, int H) {
  constexpr int BV = 16 * NCT;
  constexpr int NVT = VD / BV;
  constexpr int LDK = KD + 8;
  constexpr int RT = 8 / NW;
  __shared__ bf16 sT[2][BV][LDK];               // bf16 state, transposed: B operand of A_c S
  // consecutive logical blocks (the value tiles of one head) share an XCD, so the
  // step matrix every tile of a head reads comes from that XCD's L2 after the first
  const int logical = xcd_logical_block();
  const bool second = logical >= nb0;
  const ScanArgs p = second ? p1 : p0;
  const int blk = second ? logical - nb0 : logical;
  const int vt = blk % NVT, bh = blk / NVT;
  const int b = bh / H, h = bh % H;
  const int NT = T / C;
  const int l = lane_id(), wv = wave_id();
  const int v_base = vt * BV;
  auto rowt = [&](int i) { return wv + NW * i; };

  f32x4 st[RT][NCT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 a = zero4();
      if (p.s0) {
        const float* src = p.s0 + (size_t)bh * KD * VD;
        const int col = v_base + 16 * ct + (l & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kr = 16 * rowt(i) + 4 * (l >> 4) + r;
          a[r] = src[p.vf ? col * KD + kr : kr * VD + col];
        }
      }
      st[i][ct] = a;
    }

  bf16x8 af[D][RT][4];
  f32x4 yf[D][RT][NCT];
  f32x4 gl[D][RT];
  auto load = [&](int s, int c) {
    const size_t chh = ((size_t)b * NT + c) * H + h;
    const size_t tl = (size_t)b * T + (size_t)c * C + C - 1;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const bf16* ab = p.a + chh * A_FRAG + (size_t)(rowt(i) * 4) * 512 + l * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) af[s][i][ks] = *reinterpret_cast<const bf16x8*>(ab + ks * 512);
      const float* yb = p.y + chh * Y_FRAG + l * 4;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        yf[s][i][ct] = *reinterpret_cast<const f32x4*>(yb + (((vt * NCT + ct) * 8 + rowt(i)) * 64) * 4);
      if constexpr (GATE == AG_VECTOR) {
        gl[s][i] = *reinterpret_cast<const f32x4*>(p.g + (tl * H + h) * KD + 16 * rowt(i) + 4 * (l >> 4));
      } else if constexpr (GATE == AG_SCALAR) {
        const float x = p.g[tl * H + h];
        gl[s][i] = f32x4{x, x, x, x};
      } else {
        gl[s][i] = zero4();
      }
    }
  };
  auto publish = [&](int buf) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        bf16x4 v4;
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = to_bf16(st[i][ct][r]);
        *reinterpret_cast<bf16x4*>(&sT[buf][16 * ct + (l & 15)][16 * rowt(i) + 4 * (l >> 4)]) = v4;
      }
  };
  // Per chunk, in dependency order.  Before the barrier: the accumulator seed
  // -(lam S + Y) (own registers only).  After it: the state's B fragments from LDS,
  // the global store of S (bf16), two independent MFMA chains over K halves per
  // tile, the next loads into the slot just consumed (issued while the MFMAs run),
  // then the new state's bf16 copy into the other LDS buffer.
  f32x4 seed[RT][NCT];
  auto prepare = [&](int s) {
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      f32x4 lam;
#pragma unroll
      for (int r = 0; r < 4; ++r) lam[r] = fast_exp2(gl[s][i][r]);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) seed[i][ct][r] = -(st[i][ct][r] * lam[r] + yf[s][i][ct][r]);
    }
  };
  auto step = [&](int s, int c, int buf, int c_next) {
    bf16x8 bfr[NCT][4];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) bfr[ct][ks] = frag(&sT[buf][16 * ct][32 * ks], LDK);
    bf16* dst = p.s_out + (((size_t)b * NT + c) * H + h) * KD * VD;
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          dst[(16 * rowt(i) + 4 * (l >> 4) + r) * VD + v_base + 16 * ct + (l & 15)] = to_bf16(st[i][ct][r]);
    f32x4 a0[RT][NCT], a1[RT][NCT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        a0[i][ct] = mfma(af[s][i][0], bfr[ct][0], seed[i][ct]);
        a1[i][ct] = mfma(af[s][i][2], bfr[ct][2], zero4());
      }
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        a0[i][ct] = mfma(af[s][i][1], bfr[ct][1], a0[i][ct]);
        a1[i][ct] = mfma(af[s][i][3], bfr[ct][3], a1[i][ct]);
      }
    if (c_next >= 0) load(s, c_next);
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) st[i][ct] = -(a0[i][ct] + a1[i][ct]);
    publish(buf ^ 1);
  };

  const int dir = p.reverse ? -1 : 1;
  int c = p.reverse ? NT - 1 : 0;
  int buf = 0;
  publish(0);
  // leading NT % D chunks one at a time, then groups of D with D chunks in flight
  const int rem = NT % D;
  for (int i = 0; i < rem; ++i) {
    load(0, c);
    prepare(0);
    lds_barrier();
    step(0, c, buf, -1);
    buf ^= 1;
    c += dir;
  }
  auto clampc = [&](int x) { return x < 0 ? 0 : (x > NT - 1 ? NT - 1 : x); };
#pragma unroll
  for (int s = 0; s < D; ++s) load(s, clampc(c + dir * s));
  for (int j = rem; j < NT; j += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      prepare(s);
      lds_barrier();
      step(s, c, buf, clampc(c + dir * D));
      buf ^= 1;
      c += dir;
    }
  }
  if (p.s_final) {
    float* dst = p.s_final + (size_t)bh * KD * VD;
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kr = 16 * rowt(i) + 4 * (l >> 4) + r, col = v_base + 16 * ct + (l & 15);
          dst[p.vf ? col * KD + kr : kr * VD + col] = st[i][ct][r];
        }
  }
}

// ---------------------------------------------------------------------------
// side: out_c = D_c + sign * rowfac * (X_c S_c), chunk-parallel
// ---------------------------------------------------------------------------
struct SideArgs {
  const bf16* x;       // [B][T][H][K] token-major
  const bf16* s;       // [B][NT][H][K][V]
  const bf16* d;       // [B][T][H][V]
  const float* g;      // scalar gate (log2 cumsum) for rowfac 2^(g_last - g_t), or null
  bf16* out;           // [B][T][H][V]
  float sign;
};

struct SideSmem {
  bf16 s[KD * VD];                // state rows [k][v], swizzled: read transposed as the B operand
  float acc[C][VD + 4];
};

__global__ __launch_bounds__(512) void affine_side_kernel(SideArgs p0, SideArgs p1, int nb0, int T, int H) {
  __shared__ SideSmem sm;
  const bool second = (int)blockIdx.x >= nb0;
  const SideArgs p = second ? p1 : p0;
  const int ch = second ? (int)blockIdx.x - nb0 : (int)blockIdx.x;
  const int NT = T / C;
  const int h = ch % H, c = (ch / H) % NT, b = ch / (H * NT);
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const size_t tok0 = (size_t)b * T + (size_t)c * C;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD;
  const bf16* sg = p.s + (size_t)ch * KD * VD;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + 512 * i;
    store_tr_chunk<16>(sm.s, q >> 4, q & 15, *reinterpret_cast<const u32x4*>(sg + (size_t)q * 8));
  }
  const int rt = wv & 3;
  bf16x8 af[4];
  const bf16* xb = p.x + (tok0 + 16 * rt + (l & 15)) * rsk + (size_t)h * KD + 8 * (l >> 4);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) af[ks] = *reinterpret_cast<const bf16x8*>(xb + 32 * ks);
  lds_barrier();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ct = 4 * (wv >> 2) + j;
    f32x4 a = zero4();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) a = mfma(af[ks], frag_tr<16>(sm.s, 32 * ks, 16 * ct), a);
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.acc[16 * rt + 4 * (l >> 4) + r][16 * ct + (l & 15)] = a[r];
  }
  lds_barrier();
  const float glast = p.g ? p.g[(tok0 + C - 1) * H + h] : 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 512 * i;
    const int t = q >> 4, cc = q & 15;
    const float f = p.sign * (p.g ? fast_exp2(glast - p.g[(tok0 + t) * H + h]) : 1.f);
    const size_t o = (tok0 + t) * rsv + (size_t)h * VD + cc * 8;
    const bf16x8 dd = *reinterpret_cast<const bf16x8*>(p.d + o);
    const f32x4 a0 = *reinterpret_cast<const f32x4*>(&sm.acc[t][cc * 8]);
    const f32x4 a1 = *reinterpret_cast<const f32x4*>(&sm.acc[t][cc * 8 + 4]);
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[e] = to_bf16(to_f32(dd[e]) + f * a0[e]);
      r[e + 4] = to_bf16(to_f32(dd[e + 4]) + f * a1[e]);
    }
    *reinterpret_cast<bf16x8*>(p.out + o) = r;
  }
}

// chunks of step operands in flight per scan work-group
#ifndef REWY_SCAN_DEPTH
#define REWY_SCAN_DEPTH 4
#endif
// waves per scan work-group (8, 4 or 2)
#ifndef REWY_SCAN_WAVES
#define REWY_SCAN_WAVES 8
#endif

template <int NCT, int GATE>
static hipError_t launch_scan(const ScanArgs& a0, const ScanArgs& a1, int n, int B, int T, int H, hipStream_t s) {
  const int nb = B * H * (VD / (16 * NCT));
  constexpr int NW = REWY_SCAN_WAVES;
  hipLaunchKernelGGL((affine_scan_kernel<NCT, (NCT >= 4 ? 2 : REWY_SCAN_DEPTH), GATE, NW>), dim3(nb * n), dim3(64 * NW),
                     0, s, a0, a1, nb, T, H);
  return hipGetLastError();
}

template <int NCT>
static hipError_t launch_scan_g(int gate, const ScanArgs& a0, const ScanArgs& a1, int n, int B, int T, int H,
                                hipStream_t s) {
  switch (gate) {
    case AG_NONE: return launch_scan<NCT, AG_NONE>(a0, a1, n, B, T, H, s);
    case AG_SCALAR: return launch_scan<NCT, AG_SCALAR>(a0, a1, n, B, T, H, s);
    case AG_VECTOR: return launch_scan<NCT, AG_VECTOR>(a0, a1, n, B, T, H, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rewy

using namespace rewy;

static bool aff_dims_ok(int B, int T, int H, int K, int V, int chunk) {
  return K == KD && V == VD && chunk == C && T > 0 && T % C == 0 && B > 0 && H > 0 &&
         (long long)B * (T / C) * H < (1LL << 31);
}

template <int GATE>
static void launch_prep(const PrepArgs* bwd, const PrepArgs* fwd, int n, int T, int H, hipStream_t stream) {
  if (bwd && fwd) {
    if (bwd->aqk) hipLaunchKernelGGL((affine_prep_pair_kernel<GATE, true>), dim3(2 * n), dim3(512), 0, stream, *bwd, *fwd, n, T, H);
    else hipLaunchKernelGGL((affine_prep_pair_kernel<GATE, false>), dim3(2 * n), dim3(512), 0, stream, *bwd, *fwd, n, T, H);
  } else if (bwd) {
    if (bwd->aqk) hipLaunchKernelGGL((affine_prep_kernel<true, GATE, true>), dim3(n), dim3(512), 0, stream, *bwd, T, H);
    else hipLaunchKernelGGL((affine_prep_kernel<true, GATE, false>), dim3(n), dim3(512), 0, stream, *bwd, T, H);
  } else {
    hipLaunchKernelGGL((affine_prep_kernel<false, GATE, false>), dim3(n), dim3(512), 0, stream, *fwd, T, H);
  }
}

static hipError_t prep_dispatch(int gate_mode, const PrepArgs* bwd, const PrepArgs* fwd, int n, int T, int H,
                                hipStream_t stream) {
  switch (gate_mode) {
    case AG_NONE: launch_prep<AG_NONE>(bwd, fwd, n, T, H, stream); break;
    case AG_SCALAR: launch_prep<AG_SCALAR>(bwd, fwd, n, T, H, stream); break;
    case AG_VECTOR: launch_prep<AG_VECTOR>(bwd, fwd, n, T, H, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static bool prep_bwd_ok(const void* q, const void* k, const void* w, const void* dO, const float* aqk,
                        const void* dv_in, const void* step, const float* offset, const void* dv_out) {
  if (!q || !k || !w || !dO || !step || !offset) return false;
  if ((aqk == nullptr) == (dv_in == nullptr)) return false;
  return !(aqk && !dv_out);
}

extern "C" hipError_t fdr_affine_prep_bwd(const void* q, const void* k, const void* w, const float* g,
                                          int gate_mode, const void* dO, const float* aqk, const void* dv_in,
                                          void* a_frag, float* y_frag, void* dv_out, int B, int T, int H,
                                          int K, int V, int chunk, float scale, hipStream_t stream) {
  if (!aff_dims_ok(B, T, H, K, V, chunk)) return hipErrorInvalidValue;
  if (!prep_bwd_ok(q, k, w, dO, aqk, dv_in, a_frag, y_frag, dv_out)) return hipErrorInvalidValue;
  if (gate_mode != AG_NONE && !g) return hipErrorInvalidValue;
  const PrepArgs a{(const bf16*)q, (const bf16*)k, (const bf16*)w, g, (const bf16*)dO, aqk, (const bf16*)dv_in,
                   (bf16*)a_frag, y_frag, (bf16*)dv_out, scale};
  return prep_dispatch(gate_mode, &a, nullptr, B * (T / C) * H, T, H, stream);
}

extern "C" hipError_t fdr_affine_prep_fwd(const void* k, const void* w, const void* u, const float* g,
                                          int gate_mode, void* a_frag, float* y_frag, int B, int T, int H,
                                          int K, int V, int chunk, hipStream_t stream) {
  if (!aff_dims_ok(B, T, H, K, V, chunk)) return hipErrorInvalidValue;
  if (!k || !w || !u || !a_frag || !y_frag) return hipErrorInvalidValue;
  if (gate_mode != AG_NONE && !g) return hipErrorInvalidValue;
  const PrepArgs a{nullptr, (const bf16*)k, (const bf16*)w, g, (const bf16*)u, nullptr, nullptr,
                   (bf16*)a_frag, y_frag, nullptr, 1.f};
  return prep_dispatch(gate_mode, nullptr, &a, B * (T / C) * H, T, H, stream);
}

extern "C" hipError_t fdr_affine_prep_pair(const void* q, const void* k, const void* w, const void* u,
                                           const float* g, int gate_mode, const void* dO, const float* aqk,
                                           const void* dv_in, void* step_bwd, float* offset_bwd, void* dv_out,
                                           void* step_fwd, float* offset_fwd, int B, int T, int H, int K, int V,
                                           int chunk, float scale, hipStream_t stream) {
  if (!aff_dims_ok(B, T, H, K, V, chunk)) return hipErrorInvalidValue;
  if (!prep_bwd_ok(q, k, w, dO, aqk, dv_in, step_bwd, offset_bwd, dv_out)) return hipErrorInvalidValue;
  if (!u || !step_fwd || !offset_fwd) return hipErrorInvalidValue;
  if (gate_mode != AG_NONE && !g) return hipErrorInvalidValue;
  const PrepArgs b{(const bf16*)q, (const bf16*)k, (const bf16*)w, g, (const bf16*)dO, aqk, (const bf16*)dv_in,
                   (bf16*)step_bwd, offset_bwd, (bf16*)dv_out, scale};
  const PrepArgs f{nullptr, (const bf16*)k, (const bf16*)w, g, (const bf16*)u, nullptr, nullptr,
                   (bf16*)step_fwd, offset_fwd, nullptr, 1.f};
  return prep_dispatch(gate_mode, &b, &f, B * (T / C) * H, T, H, stream);
}

extern "C" hipError_t fdr_affine_scan(const fdr_scan_problem* probs, int n_problems, int B, int T, int H, int K,
                                      int V, int chunk, int value_block, hipStream_t stream) {
  if (!aff_dims_ok(B, T, H, K, V, chunk) || !probs || n_problems < 1 || n_problems > 2) return hipErrorInvalidValue;
  ScanArgs a[2];
  for (int i = 0; i < n_problems; ++i) {
    const fdr_scan_problem& p = probs[i];
    if (!p.step || !p.offset || !p.states) return hipErrorInvalidValue;
    if (p.gate_mode < AG_NONE || p.gate_mode > AG_VECTOR || (p.gate_mode != AG_NONE && !p.g)) return hipErrorInvalidValue;
    if (p.gate_mode != probs[0].gate_mode) return hipErrorInvalidValue;    // one gate mode per launch
    a[i] = ScanArgs{(const bf16*)p.step, p.offset, p.g, p.initial, (bf16*)p.states, p.final_state,
                    p.reverse ? 1 : 0, p.state_v_first ? 1 : 0};
  }
  if (n_problems == 1) a[1] = a[0];
  const int gate = probs[0].gate_mode;
  switch (value_block) {
    case 16: return launch_scan_g<1>(gate, a[0], a[1], n_problems, B, T, H, stream);
    case 32: return launch_scan_g<2>(gate, a[0], a[1], n_problems, B, T, H, stream);
    case 64: return launch_scan_g<4>(gate, a[0], a[1], n_problems, B, T, H, stream);
    default: return hipErrorInvalidValue;
  }
}

extern "C" hipError_t fdr_affine_side(const fdr_side_problem* probs, int n_problems, int B, int T, int H, int K,
                                      int V, int chunk, hipStream_t stream) {
  if (!aff_dims_ok(B, T, H, K, V, chunk) || !probs || n_problems < 1 || n_problems > 2) return hipErrorInvalidValue;
  SideArgs a[2];
  for (int i = 0; i < n_problems; ++i) {
    const fdr_side_problem& p = probs[i];
    if (!p.x || !p.states || !p.addend || !p.out) return hipErrorInvalidValue;
    a[i] = SideArgs{(const bf16*)p.x, (const bf16*)p.states, (const bf16*)p.addend, p.row_gate, (bf16*)p.out,
                    p.sign};
  }
  if (n_problems == 1) a[1] = a[0];
  const int nb = B * (T / C) * H;
  hipLaunchKernelGGL(affine_side_kernel, dim3(nb * n_problems), dim3(512), 0, stream, a[0], a[1], nb, T, H);
  return hipGetLastError();
}
