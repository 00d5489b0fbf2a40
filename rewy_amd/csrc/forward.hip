// Chunk-parallel pieces of the delta-rule forward.
//
// Replace, per chunk-head, the parts of FLA's chunk_kda_fwd / chunk_gdn2_fwd /
// chunk_gated_delta_rule_fwd / chunk_delta_rule_fwd (reference
// _compat/kda.py:89-113, _compat/gdn.py:33-123, _compat/gdn2.py:87-108) that
// are not the state scan:
//
//   fdr_fwd_prepare (one work-group per chunk-head):
//     gc  = chunk-local cumsum of the raw (natural-log) gate, times 1/ln 2   (FLA chunk_local_cumsum)
//     Aqk = scale tril(q k^T 2^(g_i - g_s))                                 (diagonal included)
//     Akk = (I + strict_tril((b k) k^T 2^(g_i - g_s)))^-1                  (FLA chunk_*_fwd_intra + solve_tril)
//   fdr_fwd_o (one work-group per chunk-head):
//     o   = scale (q 2^g) h_c + Aqk v_new                                   (FLA chunk_fwd_o)
//
// The state scan between them is fdr_fwd_h and the WY factors are
// fdr_prepare_wu (recompute.hip).
//
// Gate products.  For rows i of 16-row block I and rows s of block J <= I the
// per-channel factor 2^(g_i - g_s) is split at the anchor n = 16 I (the first
// row of block I): q 2^(g_i - g_n) <= 1 and k 2^(g_n - g_s) (<= 1 for J < I),
// both split into bf16 hi + lo so each 16 x 16 tile is three MFMAs per 32-wide
// slice of K (16-bit operand mantissas, the lo x lo term dropped).  A diagonal block whose gate span reaches 100 in
// log2 units (where the k-side factor could overflow) is evaluated pairwise in
// fp32 instead.
#include "common.hpp"
#include "rewy_amd.h"

namespace rewy {

enum GateModeF { FG_NONE = 0, FG_SCALAR = 1, FG_VECTOR = 2 };

namespace fwd {
constexpr int LDK = KD + 8;     // bf16 pitch of the q, k, b rows
constexpr int LDG = KD + 4;     // fp32 pitch of the gate rows
constexpr int LDM = C + 4;      // fp32 pitch of the 64 x 64 matrices
constexpr float RCP_LN2 = 1.4426950408889634f;
constexpr float WIDE = 100.f;   // diagonal-block gate span that takes the pairwise path
}  // namespace fwd

// LDS of fwd_prepare: the staged rows and gates are dead once the 16 x 16 tiles are
// formed, so the inverse's matrices reuse their bytes (KDA: 69 KiB, two work-groups per CU).
template <int GATE, bool VEC_B>
struct PrepareSmem {
  struct In {
    bf16 q[C][fwd::LDK];
    bf16 k[C][fwd::LDK];
    bf16 b[VEC_B ? C : 1][fwd::LDK];
    float g[GATE == FG_VECTOR ? C : 1][fwd::LDG];
  };
  struct Inv {
    float M[C][fwd::LDM];    // strict_tril(b k k^T 2^(g_i-g_s))
    float X[C][fwd::LDM];    // (I + M)^-1
    float T[32][36];         // products of the block inverse
  };
  union {
    In in;
    Inv inv;
  };
  float gs[C];               // scalar gate (log2 cumsum) per row
  float beta[C];
  int wide[4];               // diagonal block I takes the pairwise path
};

template <int GATE, bool VEC_B, bool MAP>
__global__ __launch_bounds__(512) void fwd_prepare_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const float* __restrict__ graw,
    const float* __restrict__ beta, const bf16* __restrict__ bgate, float* __restrict__ gc_out,
    float* __restrict__ aqk_out, float* __restrict__ akk_out, int T, int H, int HQ, float scale,
    const int* __restrict__ cu, const int* __restrict__ ci) {
  using fwd::LDG;
  using fwd::LDK;
  using fwd::LDM;
  __shared__ __attribute__((aligned(16))) PrepareSmem<GATE, VEC_B> sm;
  auto& sq = sm.in.q;
  auto& sk = sm.in.k;
  auto& sb = sm.in.b;
  auto& sg = sm.in.g;
  auto& sgs = sm.gs;
  auto& sbeta = sm.beta;
  auto& sM = sm.inv.M;
  auto& sX = sm.inv.X;
  auto& sT = sm.inv.T;
  auto& sWide = sm.wide;

  const int blk = blockIdx.x;
  const int NT = T / C;
  // heads run fastest: work-groups in flight together read neighbouring heads of
  // the same tokens, i.e. contiguous HBM rows
  const int h = blk % H;
  const int c = (blk / H) % NT;
  const int b = blk / (H * NT);
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int lc = l & 15, lg = l >> 4;
  const Rows<MAP> rw = chunk_rows<MAP>(cu, ci, b, c, T);
  const size_t tok0 = rw.tok0;
  const size_t rsk = (size_t)H * KD;
  const size_t kofs = tok0 * rsk + (size_t)h * KD;
  const size_t mofs = (tok0 * H + h) * C;      // [t][64] matrices of this chunk-head
  const size_t rsm = (size_t)H * C;
  const QKRows qr = qk_rows(tok0, h, H, HQ);   // q / k rows (grouped value heads: HQ < H)

  // ---- stage q, k (, b) rows; gate cumsum ----
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, c8 = (p & 15) * 8;
    *reinterpret_cast<u32x4*>(&sq[t][c8]) =
        *reinterpret_cast<const u32x4*>(rw.src(q + qr.ofs + (size_t)t * qr.rs + c8, t));
    *reinterpret_cast<u32x4*>(&sk[t][c8]) =
        *reinterpret_cast<const u32x4*>(rw.src(k + qr.ofs + (size_t)t * qr.rs + c8, t));
    if constexpr (VEC_B)
      *reinterpret_cast<u32x4*>(&sb[t][c8]) =
          *reinterpret_cast<const u32x4*>(rw.src(bgate + kofs + (size_t)t * rsk + c8, t));
  }
  if constexpr (!VEC_B) {
    if (tid < C) sbeta[tid] = *rw.src(beta + (tok0 + tid) * H + h, tid);
  }
  if constexpr (GATE == FG_VECTOR) {
    // four threads per channel, 16 rows each: local sums, then the carries
    const int col = tid & 127, part = tid >> 7;
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = *rw.src(graw + kofs + (size_t)(16 * part + r) * rsk + col, 16 * part + r);
#pragma unroll
    for (int r = 1; r < 16; ++r) v[r] += v[r - 1];
#pragma unroll
    for (int r = 0; r < 16; ++r) sg[16 * part + r][col] = v[r];
    lds_barrier();
    float carry = 0.f;
    for (int pp = 0; pp < part; ++pp) carry += sg[16 * pp + 15][col];
    lds_barrier();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float x = (v[r] + carry) * fwd::RCP_LN2;
      sg[16 * part + r][col] = x;
      *rw.dst(gc_out + kofs + (size_t)(16 * part + r) * rsk + col, 16 * part + r) = x;
    }
  } else if constexpr (GATE == FG_SCALAR) {
    if (wv == 0) {
      float x = *rw.src(graw + (tok0 + l) * H + h, l);
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d);
        if (l >= d) x += y;
      }
      x *= fwd::RCP_LN2;
      sgs[l] = x;
      *rw.dst(gc_out + (tok0 + l) * H + h, l) = x;
    }
  }
  lds_barrier();

  auto gate = [&](int t, int kc) -> float {
    if constexpr (GATE == FG_VECTOR) return sg[t][kc];
    else if constexpr (GATE == FG_SCALAR) return sgs[t];
    else return 0.f;
  };

  // ---- wide diagonal blocks: gate span (over any channel) >= WIDE; one wave per block ----
  // (the gates are cumsums of log decays, so a block's span is first row - last row)
  if (wv < 4) {
    const int I = wv;
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = l + 64 * j;
      m = fmaxf(m, gate(16 * I, col) - gate(16 * I + 15, col));
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
    if (l == 0) sWide[I] = m >= fwd::WIDE;
  }
  lds_barrier();

  // ---- 16 x 16 tiles (I, J), J <= I: Aqk and M by anchored MFMAs ----
  // wave -> (row block I, first column block J0, tile count): the two waves with two tiles
  // form the q / b k row operands of block I once for both; every wave has at most two.
  const int I = wv == 0 || wv == 2 || wv == 3 ? 3 : wv == 1 || wv == 4 ? 2 : wv == 7 ? 0 : 1;
  const int J0 = wv == 2 ? 2 : wv == 3 ? 3 : wv == 4 ? 2 : wv == 6 ? 1 : 0;
  const int NJ = wv < 2 ? 2 : 1;
  f32x4 mkk[2] = {zero4(), zero4()};
  {
    const bool pairwise = NJ == 1 && J0 == I && sWide[I];
    const int n = 16 * I;                       // anchor row
    f32x4 aqk[2] = {zero4(), zero4()};
    if (!pairwise) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int k0 = 32 * ks + 8 * lg;
        const int ia = 16 * I + lc;             // A rows (i)
        bf16x8 qh, ql, bh_, bl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kc = k0 + j;
          const float fa = fast_exp2(gate(ia, kc) - gate(n, kc));     // <= 1
          const float kia = to_f32(sk[ia][kc]);
          const float bia = VEC_B ? to_f32(sb[ia][kc]) : sbeta[ia];
          bf16 hh, ll;
          split_bf16(to_f32(sq[ia][kc]) * fa, hh, ll);
          qh[j] = hh;
          ql[j] = ll;
          split_bf16(bia * kia * fa, hh, ll);
          bh_[j] = hh;
          bl[j] = ll;
        }
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          if (jj >= NJ) break;                  // wave-uniform
          const int sb_ = 16 * (J0 + jj) + lc;  // B columns (s)
          bf16x8 kh, kl;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int kc = k0 + j;
            const float fb = fast_exp2(gate(n, kc) - gate(sb_, kc));  // <= 1 off the diagonal
            bf16 hh, ll;
            split_bf16(to_f32(sk[sb_][kc]) * fb, hh, ll);
            kh[j] = hh;
            kl[j] = ll;
          }
          aqk[jj] = mfma(qh, kh, aqk[jj]);
          aqk[jj] = mfma(qh, kl, aqk[jj]);
          aqk[jj] = mfma(ql, kh, aqk[jj]);
          mkk[jj] = mfma(bh_, kh, mkk[jj]);
          mkk[jj] = mfma(bh_, kl, mkk[jj]);
          mkk[jj] = mfma(bl, kh, mkk[jj]);
        }
      }
    } else {
      // exact pairwise diagonal: lane (lg, lc) owns rows 16 I + 4 lg + r, column s = 16 I + lc
      const int s = 16 * I + lc;
#pragma unroll 1
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        float a = 0.f, m = 0.f;
        if (s <= i) {
#pragma unroll 4
          for (int kc = 0; kc < KD; ++kc) {
            const float f = fast_exp2(gate(i, kc) - gate(s, kc));
            const float ks_ = to_f32(sk[s][kc]);
            a += to_f32(sq[i][kc]) * ks_ * f;
            const float bi = VEC_B ? to_f32(sb[i][kc]) : sbeta[i];
            m += bi * to_f32(sk[i][kc]) * ks_ * f;
          }
        }
        aqk[0][r] = a;
        mkk[0][r] = m;
      }
    }
    // lane: rows i = 16 I + 4 lg + r, column s = 16 J + lc
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      if (jj >= NJ) break;
      const int s = 16 * (J0 + jj) + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        *rw.dst(aqk_out + mofs + (size_t)i * rsm + s, i) = (s <= i) ? scale * aqk[jj][r] : 0.f;
      }
    }
  }
  // zero upper tiles of Aqk (J > I)
  auto upper = [](int p, int& i, int& s) {
    const int tix = p >> 8, e = p & 255;
    const int I_ = tix < 3 ? 0 : tix < 5 ? 1 : 2;
    const int J = I_ + 1 + (tix - (I_ == 0 ? 0 : I_ == 1 ? 3 : 5));
    i = 16 * I_ + (e >> 4);
    s = 16 * J + (e & 15);
  };
  for (int p = tid; p < 6 * 256; p += 512) {
    int i, s_;
    upper(p, i, s_);
    *rw.dst(aqk_out + mofs + (size_t)i * rsm + s_, i) = 0.f;
  }
  lds_barrier();                                // staged rows and gates dead: M and X take their LDS
  // M tiles from the accumulators (lane: rows i = 16 I + 4 lg + r, column s = 16 J + lc), upper tiles zero
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    if (jj >= NJ) break;
    const int s_ = 16 * (J0 + jj) + lc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * I + 4 * lg + r;
      sM[i][s_] = (s_ < i) ? mkk[jj][r] : 0.f;
    }
  }
  for (int p = tid; p < 6 * 256; p += 512) {
    int i, s_;
    upper(p, i, s_);
    sM[i][s_] = 0.f;
  }
  lds_barrier();

  // ---- inverse of the unit lower-triangular I + M (fp32) ----
  // diagonal 16 x 16 blocks by forward substitution: wave 0, lane = (block, column)
  if (wv == 0) {
    const int B4 = lg, j = lc, base = 16 * B4;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == j) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc -= sM[base + i][base + m] * x[m];
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sX[base + i][base + j] = x[i];
  }
  // zero the strictly upper blocks of the inverse
  for (int p = tid; p < 6 * 256; p += 512) {
    const int tix = p >> 8, e = p & 255;
    const int I = tix < 3 ? 0 : tix < 5 ? 1 : 2;
    const int J = I + 1 + (tix - (I == 0 ? 0 : I == 1 ? 3 : 5));
    sX[16 * I + (e >> 4)][16 * J + (e & 15)] = 0.f;
  }
  lds_barrier();
  // Off-diagonal blocks by doubling, [[A, 0], [C, D]]^-1 = [[A^-1, 0], [-D^-1 C A^-1, D^-1]]:
  // first inside the two 32 x 32 diagonal blocks, then for the 64 x 64 whole (C = M off the
  // diagonal).  Each product is spread over all 512 threads (one or two outputs each),
  // with fixed trip counts (the zero upper parts of X and M are summed as zeros) and
  // 16-byte reads of the row operand.
  auto rowdot = [&](const float* row, const float* col, int pitch, int n) -> float {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int m = 0; m < 32; m += 4) {
      if (m >= n) break;
      const f32x4 r4 = *reinterpret_cast<const f32x4*>(row + m);
      a0 += r4[0] * col[(m + 0) * pitch];
      a1 += r4[1] * col[(m + 1) * pitch];
      a0 += r4[2] * col[(m + 2) * pitch];
      a1 += r4[3] * col[(m + 3) * pitch];
    }
    return a0 + a1;
  };
  {
    // P = M_{r,r-1} X_{r-1,r-1}, r = 1, 3
    const int q2 = tid >> 8, e = tid & 255, i = e >> 4, j = e & 15;
    const int cb = 32 * q2, rb = cb + 16;
    sT[16 * q2 + i][j] = rowdot(&sM[rb + i][cb], &sX[cb][cb + j], fwd::LDM, 16);
  }
  lds_barrier();
  {
    // X_{r,r-1} = -X_{r,r} P
    const int q2 = tid >> 8, e = tid & 255, i = e >> 4, j = e & 15;
    const int rb = 32 * q2 + 16;
    sX[rb + i][rb - 16 + j] = -rowdot(&sX[rb + i][rb], &sT[16 * q2][j], 36, 16);
  }
  lds_barrier();
  // T = M_BL X_TL (rows 32..63, columns 0..31)
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int o = tid + 512 * k2, i = o >> 5, j = o & 31;
    sT[i][j] = rowdot(&sM[32 + i][0], &sX[0][j], fwd::LDM, 32);
  }
  lds_barrier();
  // X_BL = -X_BR T
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int o = tid + 512 * k2, i = o >> 5, j = o & 31;
    sX[32 + i][j] = -rowdot(&sX[32 + i][32], &sT[0][j], 36, 32);
  }
  lds_barrier();
  // ---- Akk rows -> HBM ----
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, c4 = (p & 15) * 4;
    *reinterpret_cast<f32x4*>(rw.dst(akk_out + mofs + (size_t)t * rsm + c4, t)) =
        f32x4{sX[t][c4], sX[t][c4 + 1], sX[t][c4 + 2], sX[t][c4 + 3]};
  }
}

// ------------------------------------------------------------------------------------------
// fdr_fwd_o:  o = scale (q 2^g) h_c + Aqk v_new
// ------------------------------------------------------------------------------------------
template <int GATE, bool MAP>
__global__ __launch_bounds__(512) void fwd_o_kernel(const bf16* __restrict__ q, const float* __restrict__ gc,
                                                     const float* __restrict__ aqk, const bf16* __restrict__ hst,
                                                     const bf16* __restrict__ vnew, bf16* __restrict__ o_out,
                                                     int T, int H, int HQ, float scale,
                                                     const int* __restrict__ cu, const int* __restrict__ ci) {
  // swizzled, unpadded tiles (80 KiB in all, so two work-groups share a CU)
  __shared__ __attribute__((aligned(16))) bf16 sqg[C * KD];       // scale q 2^g rows [i][k], hi
  __shared__ __attribute__((aligned(16))) bf16 sqgl[C * KD];      // lo
  __shared__ __attribute__((aligned(16))) bf16 sah[C * C];        // Aqk rows [i][s], hi
  __shared__ __attribute__((aligned(16))) bf16 sal[C * C];        // lo
  __shared__ __attribute__((aligned(16))) bf16 sv[C * VD];        // v_new rows (swizzled)
  __shared__ __attribute__((aligned(16))) bf16 shT[C * KD];       // 64 rows of h [k][v] (swizzled)
  // (q h) contracts over K = the rows of h, read transposed; h is staged in two halves.
  const int blk = blockIdx.x;
  const int NT = T / C;
  // heads run fastest: work-groups in flight together read neighbouring heads of
  // the same tokens, i.e. contiguous HBM rows
  const int h = blk % H;
  const int c = (blk / H) % NT;
  const int b = blk / (H * NT);
  const int tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int lc = l & 15, lg = l >> 4;
  const Rows<MAP> rw = chunk_rows<MAP>(cu, ci, b, c, T);
  const size_t tok0 = rw.tok0;
  const size_t rsk = (size_t)H * KD;
  const size_t kofs = tok0 * rsk + (size_t)h * KD;
  const size_t mofs = (tok0 * H + h) * C;
  const size_t rsm = (size_t)H * C;
  const size_t hoff = (((size_t)b * NT + c) * H + h) * KD * VD;

  // stage scale * q 2^g (hi/lo), Aqk (hi/lo), v_new
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 512 * i;
    const int t = p >> 4, c8 = (p & 15) * 8;
    const QKRows qr = qk_rows(tok0, h, H, HQ);
    const bf16x8 qx =
        __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(rw.src(q + qr.ofs + (size_t)t * qr.rs + c8, t)));
    bf16x8 hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f = scale;
      if constexpr (GATE == FG_VECTOR) f *= fast_exp2(gc[kofs + (size_t)rw.clamp(t) * rsk + c8 + j]);
      else if constexpr (GATE == FG_SCALAR) f *= fast_exp2(gc[(tok0 + rw.clamp(t)) * H + h]);
      bf16 hh, ll;
      split_bf16(to_f32(qx[j]) * f, hh, ll);
      hi[j] = hh;
      lo[j] = ll;
    }
    store_tr_chunk<16>(sqg, t, p & 15, __builtin_bit_cast(u32x4, hi));
    store_tr_chunk<16>(sqgl, t, p & 15, __builtin_bit_cast(u32x4, lo));
    store_tr_chunk<16>(sv, t, p & 15, *reinterpret_cast<const u32x4*>(rw.src(vnew + kofs + (size_t)t * rsk + c8, t)));
    const int c4 = (p & 15) * 4;
    // causal: pieces above the diagonal are not fetched, elements above it are zero
    f32x4 a = *reinterpret_cast<const f32x4*>(tril_src(rw.src(aqk + mofs + (size_t)t * rsm + c4, t), t, p & 15));
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = tril_elem(a[r], t, c4 + r);
    bf16x4 alo;
    const bf16x4 ahi = split_hi4(a, alo);
    *reinterpret_cast<bf16x4*>(sah + tr_off<8>(t, c4)) = ahi;
    *reinterpret_cast<bf16x4*>(sal + tr_off<8>(t, c4)) = alo;
  }
  // wave w: output rows 16 (w & 3) .. +16, columns 64 (w >> 2) .. +64 (4 tiles)
  const int I = wv & 3, cb = 64 * (wv >> 2);
  f32x4 acc[4] = {zero4(), zero4(), zero4(), zero4()};
  for (int half = 0; half < 2; ++half) {
    lds_barrier();
    // h rows [64 half .. 64 half + 64)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = tid + 512 * i;
      const int r = p >> 4, c8 = (p & 15) * 8;
      store_tr_chunk<16>(shT, r, p & 15, *reinterpret_cast<const u32x4*>(hst + hoff + (size_t)(64 * half + r) * VD + c8));
    }
    lds_barrier();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 ah = frag_row<16>(sqg, 16 * I, 64 * half + 32 * ks);
      const bf16x8 al = frag_row<16>(sqgl, 16 * I, 64 * half + 32 * ks);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const bf16x8 bh_ = frag_tr<16>(shT, 32 * ks, cb + 16 * ct);   // h rows over K, columns v
        acc[ct] = mfma(ah, bh_, acc[ct]);
        acc[ct] = mfma(al, bh_, acc[ct]);
      }
    }
  }
  // Aqk v_new: A = Aqk rows i (s-contiguous), B = v_new rows read transposed
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const bf16x8 ah = frag_row<8>(sah, 16 * I, 32 * ks);
    const bf16x8 al = frag_row<8>(sal, 16 * I, 32 * ks);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const bf16x8 bv = frag_tr<16>(sv, 32 * ks, cb + 16 * ct);
      acc[ct] = mfma(ah, bv, acc[ct]);
      acc[ct] = mfma(al, bv, acc[ct]);
    }
  }
  // lane: rows 16 I + 4 lg + r, column cb + 16 ct + lc
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *rw.dst(o_out + kofs + (size_t)(16 * I + 4 * lg + r) * rsk + cb + 16 * ct + lc, 16 * I + 4 * lg + r) =
          to_bf16(acc[ct][r]);
}

}  // namespace rewy

using namespace rewy;

// B rows of T tokens (cu == nullptr), or (cu, ci) a packed batch of NC chunks, T = NC * 64
template <bool MAP>
static hipError_t fwd_prepare_launch(const void* q, const void* k, const float* g, int gate_mode, const float* beta,
                                     const void* b_gate, float* gc, float* Aqk, float* Akk, int B, int T, int H,
                                     int qk_heads, float scale, hipStream_t stream, const int* cu, const int* ci) {
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ || (b_gate && HQ != H)) return hipErrorInvalidValue;
  if (!q || !k || !Aqk || !Akk) return hipErrorInvalidValue;
  if (gate_mode != FG_NONE && (!g || !gc)) return hipErrorInvalidValue;
  const bool vec_b = b_gate != nullptr;
  if (vec_b && gate_mode != FG_VECTOR) return hipErrorInvalidValue;
  if (!vec_b && !beta) return hipErrorInvalidValue;
  const dim3 grid(B * H * (T / C)), block(512);
#define FDR_PREP(G, VB)                                                                                 \
  hipLaunchKernelGGL((fwd_prepare_kernel<G, VB, MAP>), grid, block, 0, stream, (const bf16*)q, (const bf16*)k, \
                     g, beta, (const bf16*)b_gate, gc, Aqk, Akk, T, H, HQ, scale, cu, ci)
  if (vec_b) FDR_PREP(FG_VECTOR, true);
  else if (gate_mode == FG_VECTOR) FDR_PREP(FG_VECTOR, false);
  else if (gate_mode == FG_SCALAR) FDR_PREP(FG_SCALAR, false);
  else if (gate_mode == FG_NONE) FDR_PREP(FG_NONE, false);
  else return hipErrorInvalidValue;
#undef FDR_PREP
  return hipGetLastError();
}

template <bool MAP>
static hipError_t fwd_o_launch(const void* q, const float* gc, int gate_mode, const float* Aqk, const void* h,
                               const void* v_new, void* o, int B, int T, int H, int qk_heads, float scale,
                               hipStream_t stream, const int* cu, const int* ci) {
  const int HQ = qk_heads > 0 ? qk_heads : H;
  if (H % HQ) return hipErrorInvalidValue;
  if (!q || !Aqk || !h || !v_new || !o) return hipErrorInvalidValue;
  if (gate_mode != FG_NONE && !gc) return hipErrorInvalidValue;
  const dim3 grid(B * H * (T / C)), block(512);
#define FDR_O(G)                                                                                           \
  hipLaunchKernelGGL((fwd_o_kernel<G, MAP>), grid, block, 0, stream, (const bf16*)q, gc, Aqk, (const bf16*)h, \
                     (const bf16*)v_new, (bf16*)o, T, H, HQ, scale, cu, ci)
  if (gate_mode == FG_VECTOR) FDR_O(FG_VECTOR);
  else if (gate_mode == FG_SCALAR) FDR_O(FG_SCALAR);
  else if (gate_mode == FG_NONE) FDR_O(FG_NONE);
  else return hipErrorInvalidValue;
#undef FDR_O
  return hipGetLastError();
}

extern "C" hipError_t fdr_fwd_prepare(const void* q, const void* k, const float* g, int gate_mode,
                                      const float* beta, const void* b_gate, float* gc, float* Aqk, float* Akk,
                                      int B, int T, int H, int qk_heads, int K, int chunk, float scale,
                                      hipStream_t stream) {
  if (K != KD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  return fwd_prepare_launch<false>(q, k, g, gate_mode, beta, b_gate, gc, Aqk, Akk, B, T, H, qk_heads, scale, stream,
                                   nullptr, nullptr);
}

extern "C" hipError_t fdr_fwd_prepare_varlen(const void* q, const void* k, const float* g, int gate_mode,
                                             const float* beta, const void* b_gate, float* gc, float* Aqk,
                                             float* Akk, const int* cu_seqlens, const int* chunk_indices,
                                             int num_chunks, int H, int qk_heads, int K, int chunk, float scale,
                                             hipStream_t stream) {
  if (K != KD || chunk != C || num_chunks <= 0 || H <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return fwd_prepare_launch<true>(q, k, g, gate_mode, beta, b_gate, gc, Aqk, Akk, 1, num_chunks * C, H, qk_heads,
                                  scale, stream, cu_seqlens, chunk_indices);
}

extern "C" hipError_t fdr_fwd_o(const void* q, const float* gc, int gate_mode, const float* Aqk, const void* h,
                                const void* v_new, void* o, int B, int T, int H, int qk_heads, int K, int V,
                                int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || T <= 0 || T % C || B <= 0 || H <= 0) return hipErrorInvalidValue;
  return fwd_o_launch<false>(q, gc, gate_mode, Aqk, h, v_new, o, B, T, H, qk_heads, scale, stream, nullptr, nullptr);
}

extern "C" hipError_t fdr_fwd_o_varlen(const void* q, const float* gc, int gate_mode, const float* Aqk,
                                       const void* h, const void* v_new, void* o, const int* cu_seqlens,
                                       const int* chunk_indices, int num_chunks, int H, int qk_heads, int K, int V,
                                       int chunk, float scale, hipStream_t stream) {
  if (K != KD || V != VD || chunk != C || num_chunks <= 0 || H <= 0 || !cu_seqlens || !chunk_indices)
    return hipErrorInvalidValue;
  return fwd_o_launch<true>(q, gc, gate_mode, Aqk, h, v_new, o, 1, num_chunks * C, H, qk_heads, scale, stream,
                            cu_seqlens, chunk_indices);
}
