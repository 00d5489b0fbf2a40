// Shared device helpers for the gfx950 delta-rule backward kernels.
//
// Operand convention for every MFMA in this library: both operands are held
// "K-contiguous" in LDS, i.e. A as [M][K] and B as [N][K] with the contraction
// index innermost.  One 16-byte read per lane then yields a full 8-element
// fragment of v_mfma_f32_16x16x32_bf16 for either operand.  The accumulator
// layout is the hardware's: lane l holds column (l & 15) and rows
// 4*(l >> 4) + r, r = 0..3, of a 16x16 tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rewy {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Native vector types for 16-byte register copies: HIP's uint4 / float4 are
// structs whose copies lower to memcpy, which keeps them out of registers
// (the backend then parks them in LDS or scratch).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int C = 64;     // chunk length
constexpr int KD = 128;   // key width
constexpr int VD = 128;   // value width

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// An MFMA reads its A/B operands from all 64 lanes whatever the EXEC mask, so
// operands must never be produced under lane-divergent control flow (lanes
// that skipped the producing load would feed stale registers to every output
// column).  Branch on wave-uniform values only around MFMAs and their loads.
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// 8-element fragment of a K-contiguous tile whose row 0 / k 0 is at `base`.
__device__ __forceinline__ bf16x8 frag(const bf16* base, int ld, int l = lane_id()) {
  return *reinterpret_cast<const bf16x8*>(base + (l & 15) * ld + 8 * (l >> 4));
}

__device__ __forceinline__ bf16 to_bf16(float x) { return static_cast<bf16>(x); }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

// hi + lo split of an fp32 value into two bf16 (hi exact in bf16, lo the rest).
__device__ __forceinline__ void split_bf16(float x, bf16& hi, bf16& lo) {
  hi = to_bf16(x);
  lo = to_bf16(x - to_f32(hi));
}

// hi + lo split of four fp32 values; returns hi, writes lo.
__device__ __forceinline__ bf16x4 split_hi4(f32x4 x, bf16x4& lo) {
  bf16x4 hi;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bf16 h, l;
    split_bf16(x[r], h, l);
    hi[r] = h;
    lo[r] = l;
  }
  return hi;
}

// 2^x on the hardware transcendental unit (no denormal-range fix-up: results
// below 2^-126 flush to zero, which every use here tolerates).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Logical work-group index remapped so that consecutive logical indices stay on
// one XCD (hardware dispatches linear work-group ids round-robin over 8 XCDs,
// each with its own L2).  Identity when the grid is not a multiple of 8.
__device__ __forceinline__ int xcd_logical_block() {
  const int n = gridDim.x;
  const int b = blockIdx.x;
  if (n % 8) return b;
  return (b % 8) * (n / 8) + b / 8;
}

// q / k may have fewer heads (HQ) than the value side (H): grouped value heads, FLA's head
// map i_h = i_hv / (H / HQ).  Offset of the row of token tok0 of q / k for value head h,
// and the distance between consecutive tokens.
struct QKRows {
  size_t ofs, rs;
};
__device__ __forceinline__ QKRows qk_rows(size_t tok0, int h, int H, int HQ) {
  const size_t rs = (size_t)HQ * KD;
  return QKRows{tok0 * rs + (size_t)(h / (H / HQ)) * KD, rs};
}

// ---------------------------------------------------------------------------
// Variable-length batches packed along the token axis (B = 1) whose sequences start
// anywhere: FLA's IS_VARLEN indexing, cu_seqlens [N+1] token offsets and, for chunk c of
// the batch, chunk_indices[c] = (sequence, chunk of that sequence).  The last chunk of a
// sequence may hold fewer than 64 rows.  Its missing rows are masked: data rows load as
// zeros (from a zero page), rows of a chunk-local gate cumsum load as the last row that
// exists (the value a zero-padded row's cumsum continues with), and their stores go to a
// sink page.  The arithmetic is then exactly that of the sequence zero-padded to whole
// chunks, without the padded copy.  MAP = false is the dense layout (every chunk full),
// for which every helper is the identity.
// ---------------------------------------------------------------------------
static __device__ __attribute__((aligned(64))) uint32_t zero_page[16];   // never written
static __device__ __attribute__((aligned(64))) uint32_t sink_page[16];   // never read

// Piece (row t, columns 4 ch .. 4 ch + 3) of a lower-triangular [64][64] fp32 matrix (Aqk,
// and Akk = (I + M)^-1, zero above the diagonal): a piece wholly above the diagonal is read
// from the zero page (no HBM traffic, ~6 of its 16 KiB per chunk-head), and tril_elem /
// tril_piece zero the elements above the diagonal, the reference's causal mask on Aqk before
// its dot (kernels/kda_residual_npu_onchip.py:114); the kernels already treat Akk as lower
// triangular (they skip its upper blocks' products).
__device__ __forceinline__ const float* tril_src(const float* p, int t, int ch) {
  return 4 * ch <= t ? p : reinterpret_cast<const float*>(zero_page);
}
__device__ __forceinline__ float tril_elem(float x, int t, int col) { return col <= t ? x : 0.f; }
__device__ __forceinline__ f32x4 tril_piece(f32x4 a, int t, int ch) {
#pragma unroll
  for (int r = 0; r < 4; ++r) a[r] = tril_elem(a[r], t, 4 * ch + r);
  return a;
}

template <bool MAP>
struct Rows {
  size_t tok0;   // token of row 0
  int n;         // rows that exist (C unless MAP)
  __device__ __forceinline__ bool ok(int t) const {
    if constexpr (MAP) return t < n;
    else return true;
  }
  __device__ __forceinline__ int clamp(int t) const {
    if constexpr (MAP) return t < n ? t : n - 1;
    else return t;
  }
  // address of row t's element p for a load (the zero page for a missing row)
  template <class X>
  __device__ __forceinline__ const X* src(const X* p, int t) const {
    if constexpr (MAP) return t < n ? p : reinterpret_cast<const X*>(zero_page);
    else return p;
  }
  // address of row t's element p for a store (the sink page for a missing row)
  template <class X>
  __device__ __forceinline__ X* dst(X* p, int t) const {
    if constexpr (MAP) return t < n ? p : reinterpret_cast<X*>(sink_page);
    else return p;
  }
};

// Rows of chunk c of batch row b (dense: T tokens per row), or (MAP) of chunk c of the
// packed batch
template <bool MAP>
__device__ __forceinline__ Rows<MAP> chunk_rows(const int* cu, const int* ci, int b, int c, int T) {
  if constexpr (MAP) {
    const int s = ci[2 * c], j = ci[2 * c + 1];
    const int t0 = cu[s] + C * j;
    return Rows<MAP>{(size_t)t0, min(C, cu[s + 1] - t0)};
  } else {
    return Rows<MAP>{(size_t)b * T + (size_t)c * C, C};
  }
}

// Rows of chunk j of sequence s of a packed batch: on 64-token boundaries
// (cu == nullptr: the sequence's chunk j is batch chunk cglob) or (MAP) from cu_seqlens
template <bool MAP>
__device__ __forceinline__ Rows<MAP> seq_chunk_rows(const int* cu, int s, int j, int cglob) {
  if constexpr (MAP) {
    const int t0 = cu[s] + C * j;
    return Rows<MAP>{(size_t)t0, min(C, cu[s + 1] - t0)};
  } else {
    return Rows<MAP>{(size_t)cglob * C, C};
  }
}

// e^x on the hardware exp2 unit
__device__ __forceinline__ float exp_f(float x) { return fast_exp2(x * 1.4426950408889634f); }
// softplus(x) = log(1 + e^x) from y = e^x: torch's threshold (x > 20 returns x), log1p's
// accuracy for small y from its series (y < 2^-12: relative error < 2^-37), else log2(1 + y)
__device__ __forceinline__ float softplus_y(float x, float y) {
  if (x > 20.f) return x;
  if (y < 2.44140625e-4f) return y * (1.f - 0.5f * y);
  return __builtin_amdgcn_logf(1.f + y) * 0.6931471805599453f;
}
// sigmoid(x) = 1 / (1 + e^-x) from y = e^x (y = inf -> 1, y = 0 -> 0)
__device__ __forceinline__ float sigmoid_y(float y) { return 1.f / (1.f + 1.f / y); }

// Redefines a register in place (an empty asm that reads and writes it).  A value
// loaded for the next loop iteration is settled at the end of the current one,
// after that iteration's stores are issued: the compiler then waits for the load
// there, with an exact vector-memory count, instead of at the first use after the
// loop back-edge, where its count merge can degrade to vmcnt(0) and also wait for
// every store.
template <class T>
__device__ __forceinline__ void settle(T& x) { asm volatile("" : "+v"(x) : : "memory"); }

// Work-group barrier that orders LDS only.  __syncthreads() fences every
// address space, which makes each wave wait for all of its outstanding global
// loads and stores (vmcnt 0) before the barrier; kernels whose waves share
// only LDS use this one so that prefetches and output stores stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// DPP lane moves inside rows of 16 lanes: no LDS traffic, no address registers.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// value of lane `src` (any lane of the wave)
__device__ __forceinline__ float lane_read(float x, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, x)));
}

// value of lane l ^ 16
__device__ __forceinline__ float lane_xor16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}

// Sum over the 4 lane groups (lanes l, l^16, l^32, l^48) of a wave.
__device__ __forceinline__ float sum_lane_groups(float x, int l = lane_id()) {
  // xor 16 inside each 32-lane half (ds_swizzle bit mode: and 0x1f, xor 0x10)
  x += lane_xor16(x);
  x += lane_read(x, l ^ 32);
  return x;
}

// Sum over the 16 lanes of one lane group (the 16 columns of a C tile row):
// pairs, quads (quad_perm), then halves of 8 (row_half_mirror) and of 16
// (row_mirror); every lane ends with the full sum.
__device__ __forceinline__ float sum_row16(float x) {
  x += dpp_mov<0xB1>(x);    // quad_perm [1, 0, 3, 2]
  x += dpp_mov<0x4E>(x);    // quad_perm [2, 3, 0, 1]
  x += dpp_mov<0x141>(x);   // row_half_mirror
  x += dpp_mov<0x140>(x);   // row_mirror
  return x;
}

// ---------------------------------------------------------------------------
// Row-major LDS tiles read transposed.
//
// gfx950's ds_read_b64_tr_b16 lets each lane of a 16-lane group name an 8-byte
// piece (4 bf16) and returns the group's 16 x 4 pieces transposed: lane i gets
// element (i & 3) of the pieces named by lanes 4j + (i >> 2), j = 0..3.  With
// lane s naming row r0 + (s >> 2), columns c0 + 4 (s & 3) .. +3 of a row-major
// tile X[r][c], lane i receives X[r0 + j][c0 + i] for j = 0..3: four
// consecutive rows of one column, i.e. an MFMA operand fragment whose
// contraction index runs down the rows.  Token-major inputs can therefore be
// staged exactly as they sit in HBM (coalesced 16-byte rows, one ds_write_b128
// per piece) and still feed contractions over tokens.
//
// Tiles of CH 16-byte chunks per row are stored without padding; chunk c of
// row r sits at chunk c ^ tr_swz<CH>(r).  The swizzle keeps the two chunks a
// 16-lane group reads per row in one aligned pair (the pair index is XORed, the
// chunk inside the pair at most swapped) and spreads the 8 rows one half-wave
// reads (r0 + {0..3, 8..11} + 16 q) over distinct banks.  For CH = 16 it also
// maps the same chunk of 16 consecutive rows to 16 distinct chunks, so row
// fragments (frag_row: one 16-byte read per lane, 16 rows) are conflict-free too.
template <int CH>
__device__ __forceinline__ int tr_swz(int r) {
  if constexpr (CH >= 16) return (2 * (r & 3)) | ((r >> 2) & 1) | (((r >> 3) & 1) << 3);
  else if constexpr (CH == 8) return 2 * (((r >> 1) & 1) | (((r >> 3) & 1) << 1));
  else if constexpr (CH == 4) return 2 * ((r >> 3) & 1);
  else return 0;
}

// element offset of (row r, column col) in a swizzled tile of CH chunks per row
template <int CH>
__device__ __forceinline__ int tr_off(int r, int col) {
  return r * (CH * 8) + (((col >> 3) ^ tr_swz<CH>(r)) << 3) + (col & 7);
}

__device__ __forceinline__ bf16x4 ds_read_tr4(const bf16* p) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// The fragment helpers take the lane index as a defaulted argument so that a
// persistent kernel can pass a per-iteration value (keeping the address
// arithmetic inside its loop instead of hoisted and held in registers).

// Operand fragment of a contraction over rows r0 .. r0 + 31 of a swizzled
// row-major tile, for the 16 columns c0 .. c0 + 15 (lane l: column c0 + (l & 15),
// rows r0 + 8 (l >> 4) .. + 7).  Serves as the A operand of X^T Y (output
// rows = columns of X) and as the B operand of X^T Y (output columns =
// columns of Y).
template <int CH>
__device__ __forceinline__ bf16x8 frag_tr(const bf16* tile, int r0, int c0, int l = lane_id()) {
  const int i = l & 15;
  const int r = r0 + 8 * (l >> 4) + (i >> 2);
  const int col = c0 + 4 * (i & 3);
  const bf16x4 a = ds_read_tr4(tile + tr_off<CH>(r, col));
  const bf16x4 b = ds_read_tr4(tile + tr_off<CH>(r + 4, col));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// The same fragment from a padded row-major tile of pitch ld elements.
__device__ __forceinline__ bf16x8 frag_tr_pitch(const bf16* tile, int ld, int r0, int c0, int l = lane_id()) {
  const int i = l & 15;
  const int r = r0 + 8 * (l >> 4) + (i >> 2);
  const int col = c0 + 4 * (i & 3);
  const bf16x4 a = ds_read_tr4(tile + r * ld + col);
  const bf16x4 b = ds_read_tr4(tile + (r + 4) * ld + col);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Rows r0 .. r0 + 7 of column c0 + (l & 15) of a padded row-major tile of pitch ld elements
// (r0 may differ between the four 16-lane groups): the 16-byte piece a lane stores when a
// tile held transposed in LDS goes out row by row, two transposed reads instead of eight
// 2-byte ones.
__device__ __forceinline__ bf16x8 col8_tr(const bf16* tile, int ld, int r0, int c0, int l = lane_id()) {
  const int i = l & 15;
  const int r = r0 + (i >> 2);
  const int col = c0 + 4 * (i & 3);
  const bf16x4 a = ds_read_tr4(tile + r * ld + col);
  const bf16x4 b = ds_read_tr4(tile + (r + 4) * ld + col);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Row fragment of a swizzled tile: lane l reads row r0 + (l & 15), columns
// c0 + 8 (l >> 4) .. + 7 (the A/B operand layout of the K = 32 MFMA with the
// contraction running along the row).
template <int CH>
__device__ __forceinline__ bf16x8 frag_row(const bf16* tile, int r0, int c0, int l = lane_id()) {
  return *reinterpret_cast<const bf16x8*>(tile + tr_off<CH>(r0 + (l & 15), c0 + 8 * (l >> 4)));
}

// Direct HBM -> LDS copy of 16 bytes per lane (gfx950 global_load_lds_dwordx4):
// lane l's bytes land at lds_block + 16 l, lds_block wave-uniform (it goes to M0).
// Written as asm so that the compiler does not track it: it would otherwise order
// later LDS writes, and after a handful of copies every LDS access, behind all
// outstanding copies.  The caller waits for the copy explicitly (vmcnt) before the
// barrier that publishes it; the compiler's own vmcnt waits stay correct, only
// more conservative, since completion is in order.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)(const __attribute__((address_space(3))) char*)p;
}
__device__ __forceinline__ void dma16(const void* src, const void* lds_block) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr(lds_block)))
               : "memory");
}

// Direct HBM -> LDS copy of rows r0 .. r0 + 3 of a [.][128] bf16 tile whose rows
// sit `ld` elements apart in HBM, into the swizzled CH = 16 layout: lane l fetches
// the HBM chunk that the swizzle places at byte 16 l of the 1 KiB block of rows
// r0 .. r0 + 3.  r0 must be wave-uniform.
__device__ __forceinline__ void dma_rows4(bf16* tile, int r0, const bf16* src, size_t ld, int l = lane_id()) {
  const int r = r0 + (l >> 4);
  dma16(src + (size_t)r * ld + 8 * ((l & 15) ^ tr_swz<16>(r)), tile + r0 * 128);
}

// 16-byte piece (8 bf16) of row r, chunk c of a swizzled tile
template <int CH>
__device__ __forceinline__ void store_tr_chunk(bf16* tile, int r, int c, u32x4 v) {
  *reinterpret_cast<u32x4*>(tile + r * (CH * 8) + ((c ^ tr_swz<CH>(r)) << 3)) = v;
}

// 8 bf16 of a 16-byte piece, each multiplied by `s` (row scaling on staging)
__device__ __forceinline__ u32x4 scale_bf16x8(u32x4 v, float s) {
  bf16x8 x = __builtin_bit_cast(bf16x8, v);
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = to_bf16(to_f32(x[j]) * s);
  return __builtin_bit_cast(u32x4, x);
}

}  // namespace rewy
