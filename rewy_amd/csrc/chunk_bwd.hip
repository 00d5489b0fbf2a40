// Chunk-parallel part of the delta-rule backward: residual-WY local products,
// matrix intra (KDA/GDN2 vector gates, Gram-free scalar-gate form for GDN and
// DeltaNet), state-gradient epilogue and the in-chunk reverse gate cumsum, fused
// into one work-group per (chunk, head).
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
// Vector gates: the 2^(g_i-g_s) factors are applied through one anchor per
// 16-row block (the block's gate centre when its span is < 80, in log2 units,
// else the block's own top/bottom with an exact pairwise diagonal), the same
// safety rule as the reference (endpoint_intra.py:98-102).  The intra operands
// are split into bf16 hi + lo so each contraction runs as three bf16 MFMAs
// with fp32 accumulation (the reference uses tf32x3 dots for these).
#include "common.hpp"

namespace rewy {

enum GateModeC { CG_NONE = 0, CG_SCALAR = 1, CG_VECTOR = 2 };

namespace post {
constexpr int LDT = 72;    // bf16 pitch of [.][64] tiles
constexpr int LDV = 136;   // bf16 pitch of [.][128] tiles
constexpr int LDG = 68;    // fp32 pitch of [128][64] gate tile
// region A: phase 1 {A^T hi, A^T lo, dR^T}; phase 2+ {L hi, L lo, D hi, D lo}
constexpr int OFF_AKTH = 0;
constexpr int OFF_AKTL = OFF_AKTH + C * LDT * 2;
constexpr int OFF_DRT = OFF_AKTL + C * LDT * 2;
constexpr int OFF_LH = 0;
constexpr int OFF_LL = OFF_LH + C * LDT * 2;
constexpr int OFF_DH = OFF_LL + C * LDT * 2;
constexpr int OFF_DL = OFF_DH + C * LDT * 2;
constexpr int REGION_A = (OFF_DRT + KD * LDT * 2) > (OFF_DL + C * LDT * 2) ? (OFF_DRT + KD * LDT * 2)
                                                                           : (OFF_DL + C * LDT * 2);
// region B: phases 1-3 {P, R, dO}; phases 4+ {q^T, k^T, g^T, b^T}
constexpr int OFF_P = REGION_A;
constexpr int OFF_R = OFF_P + C * LDV * 2;
constexpr int OFF_DO = OFF_R + C * LDV * 2;
constexpr int END_B1 = OFF_DO + C * LDV * 2;
constexpr int OFF_QT = REGION_A;
constexpr int OFF_KT = OFF_QT + KD * LDT * 2;
constexpr int OFF_GT = OFF_KT + KD * LDT * 2;
constexpr int OFF_BT = OFF_GT + KD * LDG * 4;        // used by the vector-b family only
}  // namespace post

template <int GATE, bool VEC_B>
struct PostLayout {
  static constexpr int END_B2 = post::OFF_BT + (VEC_B ? KD * post::LDT * 2 : 0);
  static constexpr int END_B = END_B2 > post::END_B1 ? END_B2 : post::END_B1;
  static constexpr int OFF_SMALL = END_B;
  // small arrays (floats)
  static constexpr int S_BETA = 0, S_G = 64, S_DBA = 128, S_DBB = 192, S_DG = 256, S_COL = 320,
                       S_TOT = 448, S_GL = 576, S_FLAG = 704, S_N = 708;
  static constexpr int BYTES = OFF_SMALL + S_N * 4;
};

template <int GATE, bool VEC_B>
__global__ __launch_bounds__(512) void chunk_bwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ vnew, const bf16* __restrict__ dO, const bf16* __restrict__ dR,
    const float* __restrict__ g, const float* __restrict__ beta, const bf16* __restrict__ bgate,
    const bf16* __restrict__ wgate, const float* __restrict__ akk, const bf16* __restrict__ hst,
    const bf16* __restrict__ dhst, bf16* __restrict__ dq_out, bf16* __restrict__ dk_out,
    bf16* __restrict__ dv_out, float* __restrict__ dg_out, float* __restrict__ dbeta_out,
    bf16* __restrict__ db_out, bf16* __restrict__ dw_out, int T, int H, float scale) {
  using LY = PostLayout<GATE, VEC_B>;
  using namespace post;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* akTh = reinterpret_cast<bf16*>(smem + OFF_AKTH);
  bf16* akTl = reinterpret_cast<bf16*>(smem + OFF_AKTL);
  bf16* drT = reinterpret_cast<bf16*>(smem + OFF_DRT);
  bf16* Lh = reinterpret_cast<bf16*>(smem + OFF_LH);
  bf16* Ll = reinterpret_cast<bf16*>(smem + OFF_LL);
  bf16* Dh = reinterpret_cast<bf16*>(smem + OFF_DH);
  bf16* Dl = reinterpret_cast<bf16*>(smem + OFF_DL);
  bf16* sP = reinterpret_cast<bf16*>(smem + OFF_P);
  bf16* sR = reinterpret_cast<bf16*>(smem + OFF_R);
  bf16* sdO = reinterpret_cast<bf16*>(smem + OFF_DO);
  bf16* qT = reinterpret_cast<bf16*>(smem + OFF_QT);
  bf16* kT = reinterpret_cast<bf16*>(smem + OFF_KT);
  float* gT = reinterpret_cast<float*>(smem + OFF_GT);
  bf16* bT = reinterpret_cast<bf16*>(smem + OFF_BT);
  float* small = reinterpret_cast<float*>(smem + LY::OFF_SMALL);
  float* sBeta = small + LY::S_BETA;   // scalar beta per row
  float* sG = small + LY::S_G;         // scalar gate per row (log2)
  float* sDbA = small + LY::S_DBA;     // sum_v P R           (beta != 0 rows)
  float* sDbB = small + LY::S_DBB;     // direct dbeta terms  (beta ~ 0 rows)
  float* sDg = small + LY::S_DG;       // scalar gate: dG row sums
  float* sCol = small + LY::S_COL;     // [128] column partials from the upper row half
  float* sTot = small + LY::S_TOT;     // [128] column totals of the lower row half
  float* sGl = small + LY::S_GL;       // [128] last-row gate (log2) per column

  const int NT = T / C;
  const int blk = blockIdx.x;
  const int c = blk % NT;
  const int bh = blk / NT;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int cs = wv & 3;          // column strip: k (or v) in [32 cs, 32 cs + 32)
  const int rh = wv >> 2;         // row half: rows [32 rh, 32 rh + 32)
  const size_t tok0 = (size_t)b * T + (size_t)c * C;
  const size_t rsk = (size_t)H * KD, rsv = (size_t)H * VD, rsa = (size_t)H * C;
  const size_t hoff = (((size_t)b * NT + c) * H + h) * KD * VD;
  const int lc = l & 15, lg = l >> 4;

  // ---------------- phase 0: stage A^T (hi/lo), dR^T, R, dO, beta, gates ----------------
  int any_fb = 0;
  {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;                    // 1024 pieces each
      const int s = p >> 4, c0 = (p & 15) * 4;        // A: row s, 4 floats of t
      const float4 a4 = *reinterpret_cast<const float4*>(akk + (tok0 + s) * rsa + (size_t)h * C + c0);
      const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16 hi, lo;
        split_bf16(av[j], hi, lo);
        akTh[(c0 + j) * LDT + s] = hi;
        akTl[(c0 + j) * LDT + s] = lo;
      }
      const int t = p >> 4, v0 = (p & 15) * 8;        // dR/R/dO: row t, 8 bf16 of v
      const size_t off = (tok0 + t) * rsv + (size_t)h * VD + v0;
      const uint4 d4 = *reinterpret_cast<const uint4*>(dR + off);
      const bf16* pd = reinterpret_cast<const bf16*>(&d4);
#pragma unroll
      for (int j = 0; j < 8; ++j) drT[(v0 + j) * LDT + t] = pd[j];
      *reinterpret_cast<uint4*>(sR + t * LDV + v0) = *reinterpret_cast<const uint4*>(vnew + off);
      *reinterpret_cast<uint4*>(sdO + t * LDV + v0) = *reinterpret_cast<const uint4*>(dO + off);
    }
    int fb = 0;
    if (tid < C) {
      const size_t row = (tok0 + tid) * H + h;
      if constexpr (!VEC_B) {
        const float be = beta[row];
        sBeta[tid] = be;
        fb = fabsf(be) < 1e-6f;
      }
      if constexpr (GATE == CG_SCALAR) sG[tid] = g[row];
      sDbA[tid] = 0.f;
      sDbB[tid] = 0.f;
      sDg[tid] = 0.f;
    }
    if (tid < KD) {
      float gl = 0.f;
      if constexpr (GATE == CG_VECTOR) gl = g[((tok0 + C - 1) * H + h) * KD + tid];
      else if constexpr (GATE == CG_SCALAR) gl = g[(tok0 + C - 1) * H + h];
      sGl[tid] = gl;
    }
    any_fb = __syncthreads_or(fb);   // block-uniform: some row has |beta| < 1e-6
  }
  const bool has_fb = !VEC_B && any_fb != 0;

  // ---------------- phase 1: P = A^T dR ; dv ; sum_v P R ----------------
  {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int I = 2 * rh + rt;               // row tile (t)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int vcol0 = 32 * cs + 16 * ct;
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks == 0 && rh == 1) continue;    // A^T upper triangular: s < 32 <= t vanishes
          const bf16x8 bd = frag(drT + vcol0 * LDT + 32 * ks, LDT);
          acc = mfma(frag(akTh + (16 * I) * LDT + 32 * ks, LDT), bd, acc);
          acc = mfma(frag(akTl + (16 * I) * LDT + 32 * ks, LDT), bd, acc);
        }
        const int vv = vcol0 + lc;
        float rowpr[4], rowpv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * I + 4 * lg + r;
          const float pv = acc[r];
          const bf16 pb = to_bf16(pv);
          sP[t * LDV + vv] = pb;
          const size_t off = (tok0 + t) * rsv + (size_t)h * VD + vv;
          if constexpr (VEC_B) {
            const float wg = to_f32(wgate[off]);
            dv_out[off] = to_bf16(wg * pv);
            dw_out[off] = to_bf16(to_f32(v[off]) * pv);
            rowpr[r] = rowpv[r] = 0.f;
          } else {
            dv_out[off] = to_bf16(sBeta[t] * pv);
            rowpr[r] = pv * to_f32(sR[t * LDV + vv]);
            rowpv[r] = has_fb ? pv * to_f32(v[off]) : 0.f;
          }
        }
        if constexpr (!VEC_B) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float a = sum_row16(rowpr[r]);
            const float bsum = sum_row16(rowpv[r]);
            if (lc == 0) {
              const int t = 16 * I + 4 * lg + r;
              atomicAdd(&sDbA[t], a);
              if (has_fb) atomicAdd(&sDbB[t], bsum);
            }
          }
        }
      }
    }
  }
  __syncthreads();

  // prefetch state tiles for phase 3 (B operands straight from global)
  bf16x8 fh[2][4], fdh[2][4];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const size_t o = hoff + (size_t)(32 * cs + 16 * ct + lc) * VD + 32 * ks + 8 * lg;
      fh[ct][ks] = *reinterpret_cast<const bf16x8*>(hst + o);
      fdh[ct][ks] = *reinterpret_cast<const bf16x8*>(dhst + o);
    }

  // ---------------- phase 2: L = scale tril(dO R^T), D = -strict_tril(P R^T) ----------------
  {
    const int I = wv >> 1;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int J = 2 * (wv & 1) + jj;
      f32x4 aL = zero4(), aD = zero4();
      if (J <= I) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 br = frag(sR + (16 * J) * LDV + 32 * ks, LDV);
          aL = mfma(frag(sdO + (16 * I) * LDV + 32 * ks, LDV), br, aL);
          aD = mfma(frag(sP + (16 * I) * LDV + 32 * ks, LDV), br, aD);
        }
      }
      const int s = 16 * J + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        float lv = (i >= s) ? scale * aL[r] : 0.f;
        float dv_ = (i > s) ? -aD[r] : 0.f;
        if constexpr (GATE == CG_SCALAR) {
          const float f = (i >= s) ? fast_exp2(sG[i] - sG[s]) : 0.f;
          lv *= f;
          dv_ *= f;
        }
        bf16 hi, lo;
        split_bf16(lv, hi, lo);
        Lh[i * LDT + s] = hi;
        Ll[i * LDT + s] = lo;
        split_bf16(dv_, hi, lo);
        Dh[i * LDT + s] = hi;
        Dl[i * LDT + s] = lo;
      }
    }
  }

  // prefetch q, k, g (and b) for the transposed staging after phase 3
  uint4 rq[2], rk[2], rb[2];
  float4 rg[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, k0 = (p & 15) * 8;
    const size_t off = (tok0 + t) * rsk + (size_t)h * KD + k0;
    rq[i] = *reinterpret_cast<const uint4*>(q + off);
    rk[i] = *reinterpret_cast<const uint4*>(k + off);
    if constexpr (VEC_B) rb[i] = *reinterpret_cast<const uint4*>(bgate + off);
  }
  if constexpr (GATE == CG_VECTOR) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 512 * i;              // 2048 pieces of 4 floats
      const int t = p >> 5, k0 = (p & 31) * 4;
      rg[i] = *reinterpret_cast<const float4*>(g + (tok0 + t) * rsk + (size_t)h * KD + k0);
    }
  }

  // ---------------- phase 3: dq_s = dO h^T, dk_s = R dh^T, dw = P h^T ----------------
  f32x4 aq[2][2], ak[2][2], aw[2][2];
  float dgk[2];
  {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float sacc = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) sacc += to_f32(fh[ct][ks][j]) * to_f32(fdh[ct][ks][j]);
      dgk[ct] = sum_lane_groups(sacc);
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int I = 2 * rh + rt;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        f32x4 x = zero4(), y = zero4(), z = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          x = mfma(frag(sdO + (16 * I) * LDV + 32 * ks, LDV), fh[ct][ks], x);
          y = mfma(frag(sR + (16 * I) * LDV + 32 * ks, LDV), fdh[ct][ks], y);
          z = mfma(frag(sP + (16 * I) * LDV + 32 * ks, LDV), fh[ct][ks], z);
        }
        aq[rt][ct] = x;
        ak[rt][ct] = y;
        aw[rt][ct] = z;
      }
    }
  }
  __syncthreads();   // P, R, dO no longer needed: region B becomes q^T, k^T, g^T (, b^T)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, k0 = (p & 15) * 8;
    const bf16* pq = reinterpret_cast<const bf16*>(&rq[i]);
    const bf16* pk = reinterpret_cast<const bf16*>(&rk[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qT[(k0 + j) * LDT + t] = pq[j];
      kT[(k0 + j) * LDT + t] = pk[j];
    }
    if constexpr (VEC_B) {
      const bf16* pb = reinterpret_cast<const bf16*>(&rb[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) bT[(k0 + j) * LDT + t] = pb[j];
    }
  }
  if constexpr (GATE == CG_VECTOR) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 512 * i;
      const int t = p >> 5, k0 = (p & 31) * 4;
      gT[(k0 + 0) * LDG + t] = rg[i].x;
      gT[(k0 + 1) * LDG + t] = rg[i].y;
      gT[(k0 + 2) * LDG + t] = rg[i].z;
      gT[(k0 + 3) * LDG + t] = rg[i].w;
    }
  }
  __syncthreads();

  // gate value at (row i, column kk)
  auto gate_at = [&](int i, int kk) -> float {
    if constexpr (GATE == CG_VECTOR) return gT[kk * LDG + i];
    else if constexpr (GATE == CG_SCALAR) return sG[i];
    else return 0.f;
  };
  auto b_at = [&](int i, int kk) -> float {
    if constexpr (VEC_B) return to_f32(bT[kk * LDT + i]);
    else return sBeta[i];
  };

  // ---------------- phase 4: state-gradient epilogue ----------------
  // after this block: aq = dq, ak = dk, aw = dG (all per element, before intra)
  float colkdk[2] = {0.f, 0.f};
  float fbrow[2][4];
  f32x4 adb[2][2];     // vector-b family: db = k exp2(g) Eb + k ue
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int I = 2 * rh + rt;
#pragma unroll
    for (int r = 0; r < 4; ++r) fbrow[rt][r] = 0.f;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int kk = 32 * cs + 16 * ct + lc;
      const float gl = sGl[kk];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        const float gi = gate_at(i, kk);
        const float gam = (GATE == CG_NONE) ? 1.f : fast_exp2(gi);
        const float kdec = (GATE == CG_NONE) ? 1.f : fast_exp2(gl - gi);
        const float qv = to_f32(qT[kk * LDT + i]);
        const float kv = to_f32(kT[kk * LDT + i]);
        const float bv = b_at(i, kk);
        const float dqv = aq[rt][ct][r] * gam * scale;
        const float dks = ak[rt][ct][r] * kdec;
        const float eb = -aw[rt][ct][r];
        const float keb = kv * gam * eb;
        aq[rt][ct][r] = dqv;
        ak[rt][ct][r] = dks + bv * gam * eb;
        aw[rt][ct][r] = qv * dqv - kv * dks + bv * keb;
        colkdk[ct] += kv * dks;
        if constexpr (VEC_B) adb[rt][ct][r] = keb;
        else fbrow[rt][r] += keb;
      }
    }
  }
  // column partial of k * dks from the upper row half -> LDS
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const float s = sum_lane_groups(colkdk[ct]);
    colkdk[ct] = s;
    if (rh == 0 && lg == 0) sCol[32 * cs + 16 * ct + lc] = s;
  }

  // ---------------- phase 5: matrix intra ----------------
  f32x4 uq[2][2], ue[2][2], uk[2][2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int I = 2 * rh + rt;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int kk = 32 * cs + 16 * ct + lc;     // this lane's column for B fragments
      float aqa = 0.f, aka = 0.f;                 // anchors (log2) for the q side / k side
      bool pair = false;
      if constexpr (GATE == CG_VECTOR) {
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const float gs = gT[kk * LDG + 16 * I + s];
          lo = fminf(lo, gs);
          hi = fmaxf(hi, gs);
        }
        pair = (hi - lo) >= 80.f;
        const float cen = 0.5f * (lo + hi);
        aqa = pair ? hi : cen;
        aka = pair ? lo : cen;
      }
      f32x4 xq = zero4(), xe = zero4(), xk = zero4();
      // uq / ue : s in [0, 16 (I+1))
      for (int ks = 0; ks <= (I >> 1); ++ks) {
        bf16x8 bh_, bl_;
        const int s0 = 32 * ks + 8 * lg;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int s = s0 + j;
          bool ok = s < 16 * (I + 1);
          if (pair && s >= 16 * I) ok = false;
          float x = 0.f;
          if (ok) {
            x = to_f32(kT[kk * LDT + s]);
            if constexpr (GATE == CG_VECTOR) x *= fast_exp2(aqa - gT[kk * LDG + s]);
          }
          bf16 hh, ll;
          split_bf16(x, hh, ll);
          bh_[j] = hh;
          bl_[j] = ll;
        }
        const bf16x8 lh = frag(Lh + (16 * I) * LDT + 32 * ks, LDT);
        const bf16x8 ll2 = frag(Ll + (16 * I) * LDT + 32 * ks, LDT);
        const bf16x8 dh2 = frag(Dh + (16 * I) * LDT + 32 * ks, LDT);
        const bf16x8 dl2 = frag(Dl + (16 * I) * LDT + 32 * ks, LDT);
        xq = mfma(lh, bh_, xq);
        xq = mfma(lh, bl_, xq);
        xq = mfma(ll2, bh_, xq);
        xe = mfma(dh2, bh_, xe);
        xe = mfma(dh2, bl_, xe);
        xe = mfma(dl2, bh_, xe);
      }
      // uk : s in [16 I, 64); A operand = L^T / D^T rows i, read transposed
      for (int ks = (I >> 1); ks < 2; ++ks) {
        bf16x8 qh, ql, eh, el;
        const int s0 = 32 * ks + 8 * lg;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int s = s0 + j;
          bool ok = s >= 16 * I;
          if (pair && s < 16 * (I + 1)) ok = false;
          float xqv = 0.f, xev = 0.f;
          if (ok) {
            float f = 1.f;
            if constexpr (GATE == CG_VECTOR) f = fast_exp2(gT[kk * LDG + s] - aka);
            xqv = to_f32(qT[kk * LDT + s]) * f;
            xev = to_f32(kT[kk * LDT + s]) * b_at(s, kk) * f;
          }
          bf16 hh, ll;
          split_bf16(xqv, hh, ll);
          qh[j] = hh;
          ql[j] = ll;
          split_bf16(xev, hh, ll);
          eh[j] = hh;
          el[j] = ll;
        }
        bf16x8 lth, ltl, dth, dtl;
        {
          const int i = 16 * I + lc;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int s = s0 + j;
            lth[j] = Lh[s * LDT + i];
            ltl[j] = Ll[s * LDT + i];
            dth[j] = Dh[s * LDT + i];
            dtl[j] = Dl[s * LDT + i];
          }
        }
        xk = mfma(lth, qh, xk);
        xk = mfma(lth, ql, xk);
        xk = mfma(ltl, qh, xk);
        xk = mfma(dth, eh, xk);
        xk = mfma(dth, el, xk);
        xk = mfma(dtl, eh, xk);
      }
      // output scaling and the exact pairwise diagonal block when the span is wide
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        const int kc = kk;
        if constexpr (GATE == CG_VECTOR) {
          const float gi = gT[kc * LDG + i];
          xq[r] *= fast_exp2(gi - aqa);
          xe[r] *= fast_exp2(gi - aqa);
          xk[r] *= fast_exp2(aka - gi);
          if (pair) {
            float pq = 0.f, pe = 0.f, pk = 0.f;
            for (int s = 16 * I; s < 16 * (I + 1); ++s) {
              const float gs = gT[kc * LDG + s];
              const float ksv = to_f32(kT[kc * LDT + s]);
              if (s <= i) {
                const float f = fast_exp2(gi - gs);
                pq += (to_f32(Lh[i * LDT + s]) + to_f32(Ll[i * LDT + s])) * ksv * f;
                if (s < i) pe += (to_f32(Dh[i * LDT + s]) + to_f32(Dl[i * LDT + s])) * ksv * f;
              }
              if (s >= i) {
                const float f = fast_exp2(gs - gi);
                const float lsi = to_f32(Lh[s * LDT + i]) + to_f32(Ll[s * LDT + i]);
                const float dsi = to_f32(Dh[s * LDT + i]) + to_f32(Dl[s * LDT + i]);
                pk += (lsi * to_f32(qT[kc * LDT + s]) + dsi * b_at(s, kc) * ksv) * f;
              }
            }
            xq[r] += pq;
            xe[r] += pe;
            xk[r] += pk;
          }
        }
      }
      uq[rt][ct] = xq;
      ue[rt][ct] = xe;
      uk[rt][ct] = xk;
    }
  }
  __syncthreads();   // sCol visible

  // ---------------- phase 6: combine, dbeta/db, last-row terms, reverse cumsum, store ----------------
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int I = 2 * rh + rt;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int kk = 32 * cs + 16 * ct + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        const float qv = to_f32(qT[kk * LDT + i]);
        const float kv = to_f32(kT[kk * LDT + i]);
        const float bv = b_at(i, kk);
        const float xq = uq[rt][ct][r], xe = ue[rt][ct][r], xk = uk[rt][ct][r];
        if constexpr (VEC_B) adb[rt][ct][r] += kv * xe;
        aq[rt][ct][r] += xq;
        ak[rt][ct][r] += bv * xe + xk;
        aw[rt][ct][r] += qv * xq + kv * (bv * xe - xk);
        if constexpr (!VEC_B) fbrow[rt][r] += xe * kv;
      }
    }
  }
  // fallback dbeta rows: direct terms sum_k (k exp2(g) Eb + k ue)
  if constexpr (!VEC_B) {
    if (has_fb) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float s = sum_row16(fbrow[rt][r]);
          if (lc == 0) atomicAdd(&sDbB[16 * (2 * rh + rt) + 4 * lg + r], s);
        }
    }
  }

  if constexpr (GATE == CG_VECTOR) {
    // last-row state terms: dG[63][kk] += exp2(g_last) sum_v h dh + sum_rows k dks
    if (rh == 1) {
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int kk = 32 * cs + 16 * ct + lc;
        const float term = fast_exp2(sGl[kk]) * dgk[ct] + colkdk[ct] + sCol[kk];
        if (lg == 3) aw[1][ct][3] += term;
      }
    }
  }

  if constexpr (GATE == CG_VECTOR) {
    // reverse cumsum over the 64 rows of each column
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float carry = 0.f;                       // total of rows below, inside this row half
#pragma unroll
      for (int rt = 1; rt >= 0; --rt) {
        f32x4& x = aw[rt][ct];
        x[2] += x[3];
        x[1] += x[2];
        x[0] += x[1];
        const float tot = x[0];                // this lane group's 4-row total
        const float t1 = __shfl(tot, (l & 15) + 16 * 1);
        const float t2 = __shfl(tot, (l & 15) + 16 * 2);
        const float t3 = __shfl(tot, (l & 15) + 16 * 3);
        float below = carry;
        if (lg < 3) below += t3;
        if (lg < 2) below += t2;
        if (lg < 1) below += t1;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] += below;
        const float t0 = __shfl(tot, (l & 15));
        carry += t0 + t1 + t2 + t3;
      }
      if (rh == 1 && lg == 0) sTot[32 * cs + 16 * ct + lc] = carry;
    }
    __syncthreads();
    if (rh == 0) {
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float add = sTot[32 * cs + 16 * ct + lc];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) aw[rt][ct][r] += add;
      }
    }
  } else if constexpr (GATE == CG_SCALAR) {
    // scalar gate: dG row sums over all 128 columns, then the last-row state term
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s = aw[rt][0][r] + aw[rt][1][r];
        s = sum_row16(s);
        if (lc == 0) atomicAdd(&sDg[16 * (2 * rh + rt) + 4 * lg + r], s);
      }
    if (rh == 1) {
      float term = 0.f;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int kk = 32 * cs + 16 * ct + lc;
        term += fast_exp2(sGl[kk]) * dgk[ct] + colkdk[ct] + sCol[kk];
      }
      term = sum_row16(term);
      if (l == 0) atomicAdd(&sDg[C - 1], term);
    }
    __syncthreads();
  }

  // stores of dq, dk (bf16) and the vector dg (fp32)
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int I = 2 * rh + rt;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int kk = 32 * cs + 16 * ct + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        const size_t off = (tok0 + i) * rsk + (size_t)h * KD + kk;
        dq_out[off] = to_bf16(aq[rt][ct][r]);
        dk_out[off] = to_bf16(ak[rt][ct][r]);
        if constexpr (GATE == CG_VECTOR) dg_out[off] = aw[rt][ct][r];
        if constexpr (VEC_B) db_out[off] = to_bf16(adb[rt][ct][r]);
      }
    }
  }
  __syncthreads();
  if (tid < C) {
    const size_t row = (tok0 + tid) * H + h;
    if constexpr (!VEC_B) {
      const float be = sBeta[tid];
      dbeta_out[row] = fabsf(be) < 1e-6f ? sDbB[tid] : sDbA[tid] / be;
    }
    if constexpr (GATE == CG_SCALAR) {
      float acc = 0.f;
      for (int s = C - 1; s >= tid; --s) acc += sDg[s];
      dg_out[row] = acc;
    }
  }
}

template <int GATE, bool VEC_B>
static hipError_t launch_post(const void* q, const void* k, const void* v, const void* vnew,
                              const void* dO, const void* dR, const float* g, const float* beta,
                              const void* bgate, const void* wgate, const float* akk, const void* h,
                              const void* dh, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                              void* db, void* dw, int B, int T, int H, float scale, hipStream_t s) {
  using LY = PostLayout<GATE, VEC_B>;
  auto kern = chunk_bwd_kernel<GATE, VEC_B>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LY::BYTES);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int grid = B * H * (T / C);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(512), LY::BYTES, s, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, (const bf16*)vnew, (const bf16*)dO, (const bf16*)dR, g, beta,
                     (const bf16*)bgate, (const bf16*)wgate, akk, (const bf16*)h, (const bf16*)dh,
                     (bf16*)dq, (bf16*)dk, (bf16*)dv, dg, dbeta, (bf16*)db, (bf16*)dw, T, H, scale);
  return hipGetLastError();
}

}  // namespace rewy

using namespace rewy;

extern "C" hipError_t fdr_chunk_bwd(const void* q, const void* k, const void* v, const void* v_new,
                                    const void* dO, const void* dR, const float* g, int gate_mode,
                                    const float* beta, const void* b_gate, const void* w_gate,
                                    const float* Akk, const void* h, const void* dh, void* dq,
                                    void* dk, void* dv, float* dg, float* dbeta, void* db, void* dw,
                                    int B, int T, int H, int K, int V, int chunk, float scale,
                                    hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0)
    return hipErrorInvalidValue;
  if (!q || !k || !v || !v_new || !dO || !dR || !Akk || !h || !dh || !dq || !dk || !dv)
    return hipErrorInvalidValue;
  const bool vec_b = b_gate != nullptr;
  if (vec_b && (!w_gate || !db || !dw)) return hipErrorInvalidValue;
  if (!vec_b && (!beta || !dbeta)) return hipErrorInvalidValue;
  if (gate_mode != CG_NONE && (!g || !dg)) return hipErrorInvalidValue;
  if (vec_b && gate_mode != CG_VECTOR) return hipErrorInvalidValue;
#define FDR_POST(G, VB)                                                                          \
  return launch_post<G, VB>(q, k, v, v_new, dO, dR, g, beta, b_gate, w_gate, Akk, h, dh, dq, dk, \
                            dv, dg, dbeta, db, dw, B, T, H, scale, stream)
  if (vec_b) { FDR_POST(CG_VECTOR, true); }
  switch (gate_mode) {
    case CG_NONE: FDR_POST(CG_NONE, false);
    case CG_SCALAR: FDR_POST(CG_SCALAR, false);
    case CG_VECTOR: FDR_POST(CG_VECTOR, false);
    default: return hipErrorInvalidValue;
  }
#undef FDR_POST
}
