/*
 * C-ABI of the MI355X (gfx950) chunked delta-rule backward library
 * (librewy_hip.so).  Plain device pointers, sizes and a hipStream_t; no torch
 * types.  Every entry point validates its arguments, enqueues work on `stream`,
 * allocates nothing, and returns hipSuccess or the first HIP error.
 *
 * Layouts are FLA's T-major layouts, which the reference keeps:
 *   q, k, w, qg, kg         bf16  [B, T, H, K]
 *   v, v_new, dO, dR, dv    bf16  [B, T, H, V]
 *   Aqk, Akk                fp32  [B, T, H, 64]   (row t holds row t mod 64 of its chunk)
 *   h, dh (per chunk)       bf16  [B, T/64, H, K, V]
 *   h0, dht, dh0            fp32  [B, H, K, V]
 *   g (vector gate)         fp32  [B, T, H, K]    chunk-local cumsum in log2 units
 *   g (scalar gate)         fp32  [B, T, H]       chunk-local cumsum in log2 units
 *   beta                    fp32  [B, T, H]
 *   b_gate / w_gate (GDN2)  bf16  [B, T, H, K] / [B, T, H, V]
 * Supported shapes: K = V = 128, chunk = 64, T a positive multiple of 64.
 * Grouped value heads (FLA's GVA, reference _compat/kda.py:485-493): where an entry point
 * takes `qk_heads` (or `k_heads`), the raw q / k (and, for scalar gates, the q / k a state
 * recurrence reads) have that many heads, [B,T,qk_heads,K], and value head h uses q / k head
 * h / (H / qk_heads); every other per-head tensor has H heads.  0 means H.  The gradients
 * dq / dk are written per value head ([B,T,H,K]); summing each group is the caller's.
 * gate_mode: 0 = none (DeltaNet), 1 = scalar (GDN), 2 = vector (KDA, GDN2).
 *
 * Variable-length batches (the `_varlen` entry points; FLA's IS_VARLEN indexing, which the
 * reference's kernels take, e.g. kernels/endpoint_intra.py:58-63): B = 1 and N sequences
 * packed along the token axis, sequence n on tokens [cu_seqlens[n], cu_seqlens[n+1]),
 * starting anywhere.  Each sequence is cut into ceil(len / 64) chunks; the batch's chunks,
 * num_chunks in all, are listed by chunk_indices[c] = (sequence, chunk of the sequence)
 * (FLA prepare_chunk_indices) and a sequence's first chunk is chunk_offsets[n] (FLA
 * prepare_chunk_offsets).  cu_seqlens, chunk_indices (int32 [num_chunks][2]) and
 * chunk_offsets (int32 [N+1]) are device memory.  Token-indexed tensors have T =
 * cu_seqlens[N] rows; per-chunk states have num_chunks chunks.  A sequence's last chunk
 * may hold fewer than 64 tokens: its missing rows read as zero (a gate cumsum's as its
 * last row) and are never written, so the results are those of the sequence zero-padded
 * to whole chunks.  An empty sequence owns no chunk.
 */
#ifndef REWY_AMD_H
#define REWY_AMD_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Reverse inter-chunk state recurrence.
 * Replaces FLA chunk_gated_delta_rule_bwd_dhu(q,k,w,do,dv,g,gk,h0,dht,scale,...)
 * -> (dh, dh0, dr) as called at reference src/fast_delta_rule/backends/backward.py:120-121,
 * and ReWY's state_bwd (src/fast_delta_rule/kernels/vector_state_gpu.py:47-67).
 *
 * For gate_mode 2, q/k are the gate-weighted qg = q*exp2(g) and
 * kg = k*exp2(g_last - g) (vector_state_gpu.py:1-6); for modes 0/1 they are the
 * raw q/k and the kernel applies the scalar gate.  Exactly one of `aqk`
 * (dv_local = Aqk^T dO is then formed in-kernel, FLA chunk_kda_bwd_dAv) or `dv`
 * (a precomputed dv_local, FLA chunk_bwd_dv_local) must be non-null.
 * dht and dh0 may be null.  value_block = 0 picks the value-tile width.  state_v_first != 0:
 * dht and dh0 are [B,H,V,K] (FLA's state_v_first layout, reference vector_state_gpu.py:24-25);
 * the per-chunk dh stays [B,T/64,H,K,V] (internal to the backward).
 */
hipError_t fdr_state_bwd(const void* q, const void* k, const void* w, const float* g,
                         int gate_mode, const void* dO, const float* aqk, const void* dv,
                         const float* dht, void* dh, void* dr, float* dh0, int state_v_first, int B,
                         int T, int H, int qk_heads, int K, int V, int chunk, float scale, int value_block,
                         hipStream_t stream);

/*
 * fdr_state_bwd over a variable-length batch (B = 1), sequence n owning chunks
 * [chunk_offsets[n], chunk_offsets[n+1]) of num_chunks; an empty sequence passes its
 * state through (dh0 = dht).  cu_seqlens null: every sequence starts on a 64-token
 * boundary, chunk c on tokens [64 c, 64 c + 64) (T = 64 num_chunks); else the sequences
 * start anywhere (the packing described at the top).  dht / dh0 are per sequence
 * [N,H,K,V]; dh is [num_chunks,H,K,V] in packed chunk order.  Replaces the reference's
 * state_bwd with cu_seqlens / chunk_offsets (kernels/vector_state_gpu.py:47-67,
 * FLA's prepare_chunk_offsets).
 */
hipError_t fdr_state_bwd_varlen(const void* q, const void* k, const void* w, const float* g, int gate_mode,
                                const void* dO, const float* aqk, const void* dv, const float* dht, void* dh,
                                void* dr, float* dh0, int state_v_first, const int* chunk_offsets,
                                const int* cu_seqlens, int N, int num_chunks, int H, int qk_heads, int K, int V,
                                int chunk, float scale, int value_block, hipStream_t stream);

/*
 * fdr_state_bwd for a vector gate with the raw q and k (qk_heads q / k heads, FLA's head map for
 * grouped value heads): qg = q 2^g and kg = k 2^(g_last - g) are formed in-kernel as each chunk
 * is staged, with fdr_prepare_wu's roundings, from the gate tile g (fp32 [B,T,H,K], log2-unit
 * chunk-local cumsum), so dh, dR and dh0 are the bits of fdr_prepare_wu's qg / kg then
 * fdr_state_bwd.  w as fdr_prepare_wu writes it, or NULL: then w = Akk (b k 2^g) is formed
 * in-kernel too, with fdr_prepare_wu's MFMA sequence and roundings, from Akk (fp32 [B,T,H,64])
 * and beta (fp32 [B,T,H], KDA) or b_gate (bf16 [B,T,H,K], GDN2; qk_heads = H) -- exactly one of
 * the two; both are ignored when w is given.  For the recompute policy's paired recurrences,
 * where fdr_prepare_wu then need not run at all.  Dv_local from aqk (fp32 [B,T,H,64]); dense
 * rows only.
 */
hipError_t fdr_state_bwd_raw_qk(const void* q, const void* k, const void* w, const float* g, const float* beta,
                                const void* b_gate, const float* Akk, const void* dO, const float* aqk,
                                const float* dht, void* dh, void* dr, float* dh0, int state_v_first, int B, int T,
                                int H, int qk_heads, int K, int V, int chunk, float scale, int value_block,
                                hipStream_t stream);

/*
 * fdr_state_bwd for long rows and few heads, in three launches with a short sequential
 * part.  Each row's chunks are split into `segments` consecutive segments; the
 * recurrence is affine in the state, so a segment maps the state at its end X to the
 * state at its start as P X + Q (P: K x K, Q: K x V, fp32):
 *   1. every segment's P and Q in parallel (the recurrence run on the identity without
 *      source terms, and on zero with them);
 *   2. per (row, head), sequentially over the row's segments from the last: the end
 *      state of each segment (dht, or zero, for the last; P X + Q of the next otherwise),
 *      and dh0;
 *   3. every segment again from its end state, writing dh and dR (fdr_state_bwd's
 *      kernel on segments).
 * Same arguments and results as fdr_state_bwd (dh0 may be null); segments in
 * [1, T/64]; value_block (0 = by the number of segment rows) is step 3's tile width.
 * `workspace` holds fdr_state_bwd_segmented_workspace_bytes(B, H, segments) bytes.
 * Replaces the reference's state recurrence (see fdr_state_bwd) where B*H work-groups
 * leave the GPU idle and the sequence is long (the reference's long-context config).
 */
size_t fdr_state_bwd_segmented_workspace_bytes(int B, int H, int segments);

hipError_t fdr_state_bwd_segmented(const void* q, const void* k, const void* w, const float* g, int gate_mode,
                                   const void* dO, const float* aqk, const void* dv, const float* dht, void* dh,
                                   void* dr, float* dh0, int state_v_first, int B, int T, int H, int K, int V, int chunk, float scale,
                                   int segments, int value_block, void* workspace, hipStream_t stream);

/*
 * Chunk-parallel backward: residual-WY products (P = A^T dR, D, E-bar),
 * dAqk, matrix intra, gate/beta epilogue and the in-chunk reverse cumsum of dg,
 * one work-group per (chunk, head).
 * Replaces, at the seams of reference backends/backward.py:18-25,44-49,
 *   chunk_kda_bwd_wy_dqkg_fused  -> LocalBetaResidual (kernels/kda_residual_local_beta.py:8-23)
 *   chunk_kda_bwd_intra          -> EndpointMatrixIntra (kernels/endpoint_intra.py:300-326)
 *   chunk_gdn2_bwd_wy_dqkg_fused -> gdn2_consumer_fp32.residual (kernels/gdn2_consumer_fp32.py:76-86)
 *   chunk_gdn2_bwd_intra         -> gdn2_consumer_fp32.matrix_intra (:89-98)
 *   scalar_liveness_gpu.adjoint  (kernels/scalar_liveness_gpu.py:87-102, GDN/DeltaNet)
 * and the dAqk output of FLA chunk_kda_bwd_dAv.
 *
 * Scalar-beta families pass beta/dbeta and null b_gate/w_gate/db/dw; GDN2
 * passes b_gate/w_gate/db/dw (bf16) and null beta/dbeta.  Outputs dq, dk, dv
 * (bf16) and db/dw (bf16) are the final gradients; dg (fp32, same shape as g)
 * is the gradient of the raw per-token gate (natural-log units), i.e. after the
 * in-chunk reverse cumsum.  dbeta (fp32) follows the reference's branch rule:
 * sum_v(P*v_new)/beta where |beta| >= 1e-6, the direct VJP otherwise
 * (kernels/kda_residual_tri_beta.py:50-60, kda_residual_local_beta_consumer.py:161-180).
 * beta_sigmoid > 0 (scalar beta only): beta was activated in the forward as
 * beta = beta_sigmoid * sigmoid(x) (use_beta_sigmoid_in_kernel, scale 2 with
 * allow_neg_eigval; reference _compat/kda.py:202-206), and dbeta is written as dL/dx;
 * 0 writes dL/dbeta.  h_v_first != 0 (gate_mode 2 only): the saved per-chunk states h are
 * [B,T/64,H,V,K], as FLA's forward saves them under state_v_first (reference
 * _compat/kda.py:485-493); dh is always this library's [B,T/64,H,K,V] from fdr_state_bwd.
 */
hipError_t fdr_chunk_bwd(const void* q, const void* k, const void* v, const void* v_new,
                         const void* dO, const void* dR, const float* g, int gate_mode,
                         const float* beta, const void* b_gate, const void* w_gate,
                         const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                         void* dv, float* dg, float* dbeta, float beta_sigmoid, void* db, void* dw,
                         int h_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk, float scale,
                         hipStream_t stream);

/*
 * KDA's kernel-level WY seam: FLA's chunk_kda_bwd_wy_dqkg_fused(q, k, v, v_new, g, beta, A,
 * h, do, dh, dv, scale) -> (dq, dk, dv2, db, dg, dA), whose kernel the reference replaces by
 * its residual producer/consumer (backends/backward.py:23-25, LocalBetaResidual,
 * kernels/kda_residual_local_beta.py:8-23; the NPU wrapper's signature at
 * kernels/kda_residual_npu_onchip.py:683-702).  Every term of fdr_chunk_bwd but the matrix
 * intra: dq, dk fp32 [B,T,H,K] (per value head), dv bf16, dg fp32 before the in-chunk
 * reverse cumsum, dbeta fp32 complete on rows with |beta| >= 1e-6 (the residual identity;
 * the direct terms on the others, which fdr_matrix_intra with beta_complete completes), and
 * dA fp32 [B,T,H,64] = D = -strict_tril(P R^T), the dAkk the intra consumes.  dR is the
 * state recurrence's dR (FLA's dv after chunk_gated_delta_rule_bwd_dhu).  Then
 * fdr_matrix_intra(..., dAqk, dA, dq, dk, dbeta, dg, beta_complete = 1) and the reverse
 * cumsum of dg give fdr_chunk_bwd's gradients.
 */
hipError_t fdr_chunk_bwd_wy(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                            const void* dR, const float* g, const float* beta, const float* Akk, const void* h,
                            const void* dh, float* dq, float* dk, void* dv, float* dbeta, float* dg, float* dA,
                            int h_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk, float scale,
                            hipStream_t stream);

/* fdr_chunk_bwd_wy over a packed variable-length batch whose sequences start anywhere (the
 * packing described at the top; the reference seam's cu_seqlens / chunk_indices,
 * kernels/kda_residual_npu_onchip.py:683-702).  h, dh are [num_chunks,H,K,V] (h [V,K] when
 * h_v_first); rows past a sequence's end are neither read nor written. */
hipError_t fdr_chunk_bwd_wy_varlen(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                   const void* dR, const float* g, const float* beta, const float* Akk,
                                   const void* h, const void* dh, float* dq, float* dk, void* dv, float* dbeta,
                                   float* dg, float* dA, int h_v_first, const int* cu_seqlens,
                                   const int* chunk_indices, int num_chunks, int H, int qk_heads, int K, int V,
                                   int chunk, float scale, hipStream_t stream);

/*
 * GDN2's kernel-level WY seam: FLA's chunk_gdn2_bwd_wy_dqkg_fused as the reference replaces it
 * (backends/backward.py:43-47: gdn2_consumer_fp32.residual, kernels/gdn2_consumer_fp32.py:76-86,
 * whose joint consumer, :8-75, the intra seam then runs).  The reference's producer computes
 * P = A^T dR, dv2 = w_gate P, dw = v P and DM = -strict_tril(P R^T); its joint consumer the
 * state terms, the gate epilogue and the matrix intra.  Here every term but the matrix intra:
 * dq, dk fp32 [B,T,H,K], dv bf16 [B,T,H,V] (complete), db fp32 [B,T,H,K] (without the intra's
 * ue k), dw bf16 [B,T,H,V] (complete), dg fp32 before the in-chunk reverse cumsum (the last-row
 * state term included), dA fp32 [B,T,H,64] = DM.  Then fdr_matrix_intra(..., b_gate, dAqk,
 * dA, dq, dk, db, dg) and the reverse cumsum of dg give fdr_chunk_bwd's gradients.  q and k
 * have one head per value head (H).
 */
hipError_t fdr_gdn2_chunk_bwd_wy(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                 const void* dR, const float* g, const void* b_gate, const void* w_gate,
                                 const float* Akk, const void* h, const void* dh, float* dq, float* dk, void* dv,
                                 float* db, void* dw, float* dg, float* dA, int h_v_first, int B, int T, int H, int K,
                                 int V, int chunk, float scale, hipStream_t stream);

/* fdr_gdn2_chunk_bwd_wy over a packed variable-length batch (gdn2_consumer_fp32.py:76-80's
 * cu_seqlens / chunk_indices), laid out as for fdr_chunk_bwd_wy_varlen. */
hipError_t fdr_gdn2_chunk_bwd_wy_varlen(const void* q, const void* k, const void* v, const void* v_new,
                                        const void* dO, const void* dR, const float* g, const void* b_gate,
                                        const void* w_gate, const float* Akk, const void* h, const void* dh,
                                        float* dq, float* dk, void* dv, float* db, void* dw, float* dg, float* dA,
                                        int h_v_first, const int* cu_seqlens, const int* chunk_indices,
                                        int num_chunks, int H, int K, int V, int chunk, float scale,
                                        hipStream_t stream);

/* fdr_chunk_bwd over a variable-length batch whose sequences start anywhere (the packing
 * described at the top; the reference's chunk-stage kernels with cu_seqlens / chunk_indices,
 * e.g. kernels/endpoint_intra.py:58-63).  h, dh are [num_chunks,H,K,V] (or [V,K]). */
hipError_t fdr_chunk_bwd_varlen(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                const void* dR, const float* g, int gate_mode, const float* beta,
                                const void* b_gate, const void* w_gate, const float* Akk, const void* h,
                                const void* dh, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                                float beta_sigmoid, void* db, void* dw, int h_v_first, const int* cu_seqlens,
                                const int* chunk_indices, int num_chunks, int H, int qk_heads, int K, int V,
                                int chunk, float scale, hipStream_t stream);

/*
 * fdr_chunk_bwd for KDA (gate_mode 2, scalar beta, [K,V] states) in the original 7-product
 * formulation of the local WY backward -- the products of reference
 * benchmarks/data/intro_graph_data.json (FLA's prepare_wy_repr_bwd /
 * chunk_kda_bwd_kernel_wy_dqkg_fused; readable port kernels/gdn_original_separate_npu.py:226-477):
 *   W-bar = -dR h^T,  E-bar = A^T W-bar,  Z-bar = A^T dR,  T = dR Z^T + W-bar E^T,
 *   J = A^T T,  D = -strict_tril(J A^T),  dbeta by its direct VJP on every row,
 * with everything else (dAqk, the matrix intra, the epilogue and the reverse cumsum) as in
 * fdr_chunk_bwd.  No counterpart in the reference as an entry point: it is the same-GPU
 * comparator of the residual formulation (same kernel, same staging), the ablation the
 * reference reports (tests/fixtures/a800_kda_timings.json).  Outputs as fdr_chunk_bwd's.
 */
hipError_t fdr_chunk_bwd_original(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                  const void* dR, const float* g, const float* beta, const float* Akk, const void* h,
                                  const void* dh, void* dq, void* dk, void* dv, float* dg, float* dbeta, int B, int T,
                                  int H, int K, int V, int chunk, float scale, hipStream_t stream);

/*
 * Recompute of the WY factors inside the backward (recompute policy).
 * Replaces FLA recompute_w_u_fwd (called at reference backends/backward.py:110-116):
 *   w = Akk (b k 2^g), u = Akk (w_gate v)            -> bf16 [B,T,H,K] / [B,T,H,V]
 * and optionally (vector gate) qg = q 2^g, kg = k 2^(g_last - g) (bf16), or
 * (scalar / no gate) the intra-chunk scores Aqk = scale tril(q k^T 2^(g_i - g_s))
 * (fp32 [B,T,H,64]) that FLA chunk_bwd_dv_local forms (backward.py:119).
 * Scalar-beta families pass beta and null b_gate/w_gate; GDN2 passes b_gate/w_gate.
 * u = nullptr writes w (and optionally qg, kg for the vector gates, Aqk for gate_mode 0 / 1)
 * only, for fdr_fwd_h_u, which forms u itself; v and w_gate are then not read.
 */
hipError_t fdr_prepare_wu(const void* q, const void* k, const void* v, const float* g,
                          int gate_mode, const float* beta, const void* b_gate, const void* w_gate,
                          const float* Akk, void* w, void* u, void* qg, void* kg, float* Aqk, int B,
                          int T, int H, int qk_heads, int K, int V, int chunk, float scale, hipStream_t stream);

/* fdr_prepare_wu over a variable-length batch whose sequences start anywhere (the packing
 * described at the top; FLA recompute_w_u_fwd with cu_seqlens / chunk_indices). */
hipError_t fdr_prepare_wu_varlen(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                                 const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                                 void* w, void* u, void* qg, void* kg, float* Aqk, const int* cu_seqlens,
                                 const int* chunk_indices, int num_chunks, int H, int qk_heads, int K, int V,
                                 int chunk, float scale, hipStream_t stream);

/*
 * Forward state scan recomputed inside the backward.
 * Replaces FLA chunk_gated_delta_rule_fwd_h(k, w, u, g, initial_state, ...) -> (h, v_new, final)
 * as called at reference backends/backward.py:117-118:
 *   h[c] = state at chunk start (bf16 [B,T/64,H,K,V]); v_new_c = u_c - w_c h_c (bf16);
 *   state <- lambda_c state + kg_c^T v_new_c;  ht = final state (fp32, may be null).
 * For gate_mode 2, `k` is the gate-weighted kg; for modes 0/1 it is the raw k.
 * state_v_first != 0: h0 and ht are [B,H,V,K]; the per-chunk h stays [B,T/64,H,K,V].
 */
hipError_t fdr_fwd_h(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                     const float* h0, void* h, void* v_new, float* ht, int state_v_first, int B, int T, int H, int k_heads,
                     int K, int V, int chunk, int value_block, hipStream_t stream);

/*
 * fdr_fwd_h over a variable-length batch, with the packing, chunk_offsets and cu_seqlens of
 * fdr_state_bwd_varlen; h0 / ht per sequence [N,H,K,V].  Replaces FLA's
 * chunk_gated_delta_rule_fwd_h with cu_seqlens (the recompute policy's call).
 */
hipError_t fdr_fwd_h_varlen(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                            const float* h0, void* h, void* v_new, float* ht, int state_v_first,
                            const int* chunk_offsets, const int* cu_seqlens, int N, int num_chunks, int H,
                            int k_heads, int K, int V, int chunk, int value_block, hipStream_t stream);

/*
 * The forward scan of fdr_fwd_h with u formed in-kernel: FLA's recompute_w_u_fwd's u
 * (u = Akk (beta v), or Akk (w_gate v) for GDN2) folded into chunk_gated_delta_rule_fwd_h
 * (reference backends/backward.py:110-118), for the recompute policy's paired recurrences,
 * where fdr_prepare_wu (with u = nullptr) writes w but not u.  k is the raw k (k_heads q/k
 * heads); a vector gate's kg = k 2^(g_last - g) is formed in-kernel with fdr_prepare_wu's
 * rounding, as fdr_state_bwd_raw_qk forms it; w as fdr_prepare_wu writes it, or NULL: then
 * w = Akk (beta k 2^g | b_gate k 2^g) is formed in-kernel too, with fdr_prepare_wu's MFMA
 * sequence and roundings (b_gate bf16 [B,T,H,K], GDN2 with k_heads = H; it is read only
 * then), and fdr_prepare_wu need not run at all.  kg (vector gate, w given; may be NULL):
 * fdr_prepare_wu's kg [B,T,H,K], read instead of formed (k is then not read) -- cheaper at narrow
 * value tiles, where every tile would form it again; v bf16 [B,T,H,V]; beta fp32 [B,T,H], or w_gate bf16 [B,T,H,V] (vector gate only);
 * Akk fp32 [B,T,H,64].  u is formed with fdr_prepare_wu's MFMA sequence and roundings, so h,
 * v_new and ht are the bits of fdr_prepare_wu + fdr_fwd_h.  value_block as for fdr_fwd_h.
 */
hipError_t fdr_fwd_h_u(const void* k, const void* kg, const void* w, const void* v, const float* g, int gate_mode,
                       const float* beta, const void* b_gate, const void* w_gate, const float* Akk, const float* h0,
                       void* h, void* v_new, float* ht, int state_v_first, int B, int T, int H, int k_heads, int K,
                       int V, int chunk, int value_block, hipStream_t stream);

/*
 * fdr_state_bwd (direct) and fdr_fwd_h_u in one launch: the reverse state recurrence and the
 * forward scan forming u, independent of each other, run side by side -- work-groups
 * [0, n) the state recurrence's, [n, 2n) the scan's, n = B H V / value_block each -- with
 * the same kernels' code, so every output is the bits of the two calls.  This build's own
 * composition (no counterpart in the reference, which runs FLA's chunk_gated_delta_rule_fwd_h
 * and its state kernel one after the other, backends/backward.py:117-121): for batch x heads
 * too small for one recurrence to fill the GPU, where two launches on two streams would pay
 * their fork and join.  Dense rows; value_block 16, 32 or 64 (required).
 *   q, k: the state recurrence's q / k -- raw (qk_heads heads) for gate_mode 0 / 1 and with
 *         raw_qk, else fdr_prepare_wu's qg / kg [B,T,H,K];
 *   k_scan: the raw k (qk_heads heads) the scan forms kg / E from; kg: fdr_prepare_wu's kg,
 *         read by the scan instead (vector gate without raw_qk; k_scan is then not read);
 *   w: fdr_prepare_wu's w, or NULL (vector gate with raw_qk: w formed in both, from beta or
 *      b_gate, as fdr_state_bwd_raw_qk / fdr_fwd_h_u form it);
 *   gate_mode 0 / 1: w given, raw_qk 0; aqk NULL (Aqk formed by the state recurrence) or
 *      fdr_prepare_wu's Aqk (read, as fdr_state_bwd reads it);
 *   gate_mode 2: aqk given; raw_qk only at value_block 64;
 *   beta fp32 [B,T,H] or GDN2's w_gate bf16 [B,T,H,V] (and b_gate when w is NULL);
 *   v, Akk, h0 (may be null), h, v_new, ht (may be null): as fdr_fwd_h_u;
 *   dO, dht (may be null), dh, dr, dh0 (may be null), scale: as fdr_state_bwd.
 */
hipError_t fdr_paired_recurrences(const void* q, const void* k, const void* w, const void* k_scan, const void* kg,
                                  const float* g, int gate_mode, const float* beta, const void* b_gate,
                                  const void* w_gate, const void* v, const float* Akk, const float* aqk,
                                  const void* dO, const float* dht, const float* h0, void* dh, void* dr, float* dh0,
                                  void* h, void* v_new, float* ht, int raw_qk, int state_v_first, int B, int T, int H,
                                  int qk_heads, int K, int V, int chunk, float scale, int value_block,
                                  hipStream_t stream);

/*
 * The recompute-policy backward of GDN (gate_mode 1) and DeltaNet (gate_mode 0) as one call:
 * fdr_prepare_wu (w; Aqk too when aqk_in_prepare != 0), fdr_paired_recurrences (value_block
 * 16, 32 or 64; the state recurrence forms Aqk itself when aqk_in_prepare == 0) and
 * fdr_chunk_bwd, enqueued on `stream` in that order -- the reference's _scalar backward,
 * backends/backward.py:96-131 (FLA recompute_w_u_fwd, chunk_gated_delta_rule_fwd_h,
 * chunk_gated_delta_rule_bwd_dhu, then the chunk stage), with the same bits as the three
 * entry points called one by one.  This build's own composition (no single counterpart in the
 * reference): for small batches, where the host time of three calls exceeds the kernels'.
 * Inputs as those entry points take them (q / k with qk_heads heads, g fp32 [B,T,H] or NULL
 * for gate_mode 0, beta fp32 [B,T,H], Akk fp32 [B,T,H,64], dht / h0 fp32 or NULL);
 * outputs dq, dk, dv bf16 [B,T,H,K|V] per value head, dg (gate_mode 1), dbeta, dh0 (may be
 * NULL) as fdr_chunk_bwd / fdr_state_bwd write them.  workspace: device memory, 256-byte
 * aligned, of at least fdr_scalar_bwd_workspace_bytes(B, T, H, K, V, chunk) bytes, holding
 * w, Aqk, dh, dR, h and v_new; two calls in flight at once need two workspaces.  Every
 * argument rule is checked before the first launch: a rejected call launches nothing.
 */
size_t fdr_scalar_bwd_workspace_bytes(int B, int T, int H, int K, int V, int chunk);
hipError_t fdr_scalar_bwd(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                          const float* beta, const float* Akk, const void* dO, const float* dht, const float* h0,
                          void* dq, void* dk, void* dv, float* dg, float* dbeta, float* dh0, void* workspace,
                          size_t workspace_bytes, float beta_sigmoid, int aqk_in_prepare, int state_v_first, int B,
                          int T, int H, int qk_heads, int K, int V, int chunk, float scale, int value_block,
                          hipStream_t stream);

/*
 * The recompute pair fdr_prepare_wu + fdr_fwd_h in one sweep.  Replaces FLA
 * recompute_w_u_fwd(k, v, beta, A, g) -> (w, u) [, qg, kg] followed by
 * chunk_gated_delta_rule_fwd_h(k, w, u, g, initial_state) -> (h, v_new, final), as called at
 * reference backends/backward.py:110-118 (GDN / DeltaNet) and :44-49 (KDA / GDN2 when the
 * forward did not save its intermediates).  Arguments as for fdr_prepare_wu (raw q / k,
 * gate_mode 0/1/2, scalar beta or GDN2's b_gate / w_gate, Akk fp32) and fdr_fwd_h (h0, h,
 * v_new, ht, state_v_first).  Writes w (bf16 [B,T,H,K], for the backward state pass), for
 * gate_mode 2 qg and kg (bf16 [B,T,H,K]; null otherwise), h, v_new and ht, each exactly as
 * the pair writes it: w and u are formed with fdr_prepare_wu's products and roundings, bit
 * for bit.  u is never written.
 */
hipError_t fdr_fwd_h_wy(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                        const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                        const float* h0, void* w, void* qg, void* kg, void* h, void* v_new, float* ht,
                        int state_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk,
                        int value_block, hipStream_t stream);

/* fdr_fwd_h_wy over a variable-length batch: packing, chunk_offsets and cu_seqlens as for
 * fdr_fwd_h_varlen (FLA recompute_w_u_fwd + chunk_gated_delta_rule_fwd_h with cu_seqlens). */
hipError_t fdr_fwd_h_wy_varlen(const void* q, const void* k, const void* v, const float* g, int gate_mode,
                               const float* beta, const void* b_gate, const void* w_gate, const float* Akk,
                               const float* h0, void* w, void* qg, void* kg, void* h, void* v_new, float* ht,
                               int state_v_first, const int* chunk_offsets, const int* cu_seqlens, int N,
                               int num_chunks, int H, int qk_heads, int K, int V, int chunk, int value_block,
                               hipStream_t stream);

/*
 * Standalone matrix intra (the intra-chunk VJP of a vector-gated chunk), in place.
 * Replaces the reference's kernel-level seam chunk_<op>_bwd_intra
 * (q, k, g, beta, dAqk, dAkk, dq, dk, db, dg) -> (dq, dk, db, dg):
 *   KDA   EndpointMatrixIntra.__call__       kernels/endpoint_intra.py:300-326
 *   GDN2  gdn2_consumer_fp32.matrix_intra    kernels/gdn2_consumer_fp32.py:89-98
 * With L = tril(dAqk) (diagonal included), D = strict_tril(dAkk) and gates g in log2
 * units (chunk-local cumsum):
 *   uq = sum_{s<=i} L_is k_s 2^(g_i-g_s),  ue = sum_{s<i} D_is k_s 2^(g_i-g_s),
 *   uk = sum_{s>=i} (L_si q_s + D_si b_s k_s) 2^(g_s-g_i)
 *   dq += uq;  dk += b ue + uk;  dg += q uq + k (b ue - uk);  db += sum_k ue k  (scalar beta,
 *   every row, or only |beta| < 1e-6 rows when beta_complete != 0, endpoint_intra.py:190-194)
 *   or db += ue k  (GDN2's vector erase gate b_gate).
 * q, k, b_gate bf16 [B,T,H,K]; g, dq, dk, dg fp32 [B,T,H,K]; beta, db fp32 [B,T,H] (scalar
 * beta) or db fp32 [B,T,H,K] (b_gate non-null, beta null); dAqk, dAkk fp32 [B,T,H,64].
 * dq, dk, db, dg are read and rewritten (the reference's dq2 aliases dq).  dg is the
 * pre-cumsum gate gradient, as at the reference seam.
 */
hipError_t fdr_matrix_intra(const void* q, const void* k, const float* g, const float* beta,
                            const void* b_gate, const float* dAqk, const float* dAkk, float* dq,
                            float* dk, float* db, float* dg, int B, int T, int H, int qk_heads, int K, int chunk,
                            int beta_complete, hipStream_t stream);

/* fdr_matrix_intra over a packed variable-length batch whose sequences start anywhere (the
 * reference seam's cu_seqlens / chunk_indices, kernels/endpoint_intra.py:318-321,
 * gdn2_consumer_fp32.py:91-94).  Rows past a sequence's end are neither read nor written. */
hipError_t fdr_matrix_intra_varlen(const void* q, const void* k, const float* g, const float* beta,
                                   const void* b_gate, const float* dAqk, const float* dAkk, float* dq, float* dk,
                                   float* db, float* dg, const int* cu_seqlens, const int* chunk_indices,
                                   int num_chunks, int H, int qk_heads, int K, int chunk, int beta_complete,
                                   hipStream_t stream);

/*
 * Forward, chunk-parallel part 1: gate cumsum and the intra-chunk matrices.
 * Replaces, per chunk-head, FLA's chunk_local_cumsum(g, scale=RCP_LN2) and the
 * chunk_<op>_fwd_intra + solve_tril pair inside chunk_kda_fwd / chunk_gdn2_fwd /
 * chunk_gated_delta_rule_fwd / chunk_delta_rule_fwd (reference _compat/kda.py:89-113,
 * _compat/gdn.py:33-123, _compat/gdn2.py:87-108):
 *   gc  = chunk-local cumsum(g) / ln 2            fp32, g's shape (g = raw natural-log decay)
 *   Aqk = scale tril(q k^T 2^(g_i - g_s))          fp32 [B,T,H,64]
 *   Akk = (I + strict_tril((b k) k^T 2^(g_i - g_s)))^-1   fp32 [B,T,H,64]
 * b is beta (fp32 [B,T,H]) or GDN2's erase gate b_gate (bf16 [B,T,H,K]); gate_mode as above
 * (g and gc null for gate_mode 0).
 */
hipError_t fdr_fwd_prepare(const void* q, const void* k, const float* g, int gate_mode,
                           const float* beta, const void* b_gate, float* gc, float* Aqk, float* Akk,
                           int B, int T, int H, int qk_heads, int K, int chunk, float scale, hipStream_t stream);

/* fdr_fwd_prepare over a variable-length batch whose sequences start anywhere (the packing
 * described at the top; FLA's chunk_local_cumsum / fwd_intra / solve_tril with cu_seqlens). */
hipError_t fdr_fwd_prepare_varlen(const void* q, const void* k, const float* g, int gate_mode, const float* beta,
                                  const void* b_gate, float* gc, float* Aqk, float* Akk, const int* cu_seqlens,
                                  const int* chunk_indices, int num_chunks, int H, int qk_heads, int K, int chunk,
                                  float scale, hipStream_t stream);

/*
 * Forward, chunk-parallel part 2: the output.  Replaces FLA's chunk_fwd_o:
 *   o_c = scale (q_c 2^gc_c) h_c + Aqk_c v_new_c      bf16 [B,T,H,V]
 * with h (bf16 [B,T/64,H,K,V]) and v_new from fdr_fwd_h and Aqk from fdr_fwd_prepare.
 */
hipError_t fdr_fwd_o(const void* q, const float* gc, int gate_mode, const float* Aqk, const void* h,
                     const void* v_new, void* o, int B, int T, int H, int qk_heads, int K, int V, int chunk,
                     float scale, hipStream_t stream);

/* fdr_fwd_o over a variable-length batch whose sequences start anywhere (the packing
 * described at the top; FLA chunk_fwd_o with cu_seqlens / chunk_indices). */
hipError_t fdr_fwd_o_varlen(const void* q, const float* gc, int gate_mode, const float* Aqk, const void* h,
                            const void* v_new, void* o, const int* cu_seqlens, const int* chunk_indices,
                            int num_chunks, int H, int qk_heads, int K, int V, int chunk, float scale,
                            hipStream_t stream);

/*
 * KDA's in-kernel gate activation (use_gate_in_kernel=True) and its backward, as the
 * reference documents them (_compat/kda.py:250-294; dA_log / ddt_bias are the extra
 * outputs of kda_backward, backends/backward.py:63-73):
 *   no lower bound:    g = -exp(A_log[h]) * softplus(g_raw + dt_bias[h,k])
 *   lower_bound, A_log: g = lower_bound * sigmoid(exp(A_log[h]) * (g_raw + dt_bias[h,k]))
 *   lower_bound only:  g = lower_bound * sigmoid(g_raw + dt_bias[h,k])
 * g_raw [B,T,H,K] fp32 (raw_is_bf16 = 0) or bf16 (1); A_log fp32 [H] (null only with a
 * lower bound); dt_bias fp32 [H*K] or null; g fp32 [B,T,H,K].  The backward takes
 * dg = dL/dg (fp32), writes dg_raw in g_raw's dtype and, where non-null, dA_log (fp32 [H])
 * and ddt_bias (fp32 [H*K]); `workspace` holds fdr_kda_gate_workspace_bytes(B,T,H,K)
 * bytes of per-block partial sums.  K must be 128.
 */
size_t fdr_kda_gate_workspace_bytes(int B, int T, int H, int K);

hipError_t fdr_kda_gate_fwd(const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
                            int has_lower_bound, float lower_bound, float* g, int B, int T, int H, int K,
                            hipStream_t stream);

hipError_t fdr_kda_gate_bwd(const float* dg, const void* g_raw, int raw_is_bf16, const float* A_log,
                            const float* dt_bias, int has_lower_bound, float lower_bound, void* dg_raw,
                            float* dA_log, float* ddt_bias, void* workspace, int B, int T, int H, int K,
                            hipStream_t stream);

/*
 * fdr_chunk_bwd for KDA (gate_mode 2, scalar beta) with the in-kernel gate's backward
 * folded into the dg stores: instead of dg it writes dg_raw = dL/dg_raw (g_raw's dtype)
 * and, where non-null, dA_log / ddt_bias, with the activation and arguments of
 * fdr_kda_gate_bwd.  `workspace` holds fdr_chunk_bwd_gate_workspace_bytes(B, T, H) bytes
 * of per-chunk partial sums.  beta_sigmoid and h_v_first as for fdr_chunk_bwd.  Replaces the chunk
 * stage plus the gate backward of the reference's kda_backward with use_gate_in_kernel
 * (backends/backward.py:63-73).
 */
size_t fdr_chunk_bwd_gate_workspace_bytes(int B, int T, int H);

hipError_t fdr_chunk_bwd_gate_fold(const void* q, const void* k, const void* v, const void* v_new, const void* dO,
                                   const void* dR, const float* g, const float* beta, const float* Akk,
                                   const void* h, const void* dh, void* dq, void* dk, void* dv, float* dbeta,
                                   float beta_sigmoid, const void* g_raw, int raw_is_bf16, const float* A_log, const float* dt_bias,
                                   int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log,
                                   float* ddt_bias, void* workspace, int h_v_first, int B, int T, int H, int qk_heads, int K, int V,
                                   int chunk,
                                   float scale, hipStream_t stream);

/*
 * fdr_chunk_bwd_gate_fold over a packed variable-length batch whose sequences start
 * anywhere (cu_seqlens, chunk_indices and num_chunks as for fdr_chunk_bwd_varlen; rows
 * past a sequence's end are neither read nor written and add nothing to dA_log /
 * ddt_bias).  `workspace` holds fdr_chunk_bwd_gate_workspace_bytes(1, 64 * num_chunks, H)
 * bytes.  Replaces the chunk stage plus the gate backward of the reference's kda_backward
 * with use_gate_in_kernel and cu_seqlens (backends/backward.py:63-73).
 */
hipError_t fdr_chunk_bwd_gate_fold_varlen(const void* q, const void* k, const void* v, const void* v_new,
                                          const void* dO, const void* dR, const float* g, const float* beta,
                                          const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                                          void* dv, float* dbeta, float beta_sigmoid, const void* g_raw,
                                          int raw_is_bf16, const float* A_log, const float* dt_bias,
                                          int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log,
                                          float* ddt_bias, void* workspace, int h_v_first, const int* cu_seqlens,
                                          const int* chunk_indices, int num_chunks, int H, int qk_heads, int K,
                                          int V, int chunk, float scale, hipStream_t stream);

/*
 * fdr_chunk_bwd_gate_fold without the workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops or harnesses that forbid hipMalloc).  The per-chunk
 * partial sums go to a fixed device array inside the library, FDR_NOALLOC_SCRATCH_BYTES
 * (16 MiB) per GPU, held until the process ends; a problem whose
 * fdr_chunk_bwd_gate_workspace_bytes(B, T, H) exceeds it is refused with
 * hipErrorInvalidValue before anything is enqueued.  The function itself calls no
 * allocator.  All calls on one GPU share that GPU's array: calls that overlap on one
 * GPU (concurrent streams or host threads) race.  Nothing in the array needs
 * clearing between calls.
 */
#define FDR_NOALLOC_SCRATCH_BYTES (16u << 20)

hipError_t fdr_chunk_bwd_gate_fold_noalloc(const void* q, const void* k, const void* v, const void* v_new,
                                           const void* dO, const void* dR, const float* g, const float* beta,
                                           const float* Akk, const void* h, const void* dh, void* dq, void* dk,
                                           void* dv, float* dbeta, float beta_sigmoid, const void* g_raw,
                                           int raw_is_bf16, const float* A_log, const float* dt_bias,
                                           int has_lower_bound, float lower_bound, void* dg_raw, float* dA_log,
                                           float* ddt_bias, int h_v_first, int B, int T, int H, int qk_heads, int K, int V, int chunk,
                                           float scale, hipStream_t stream);

/*
 * beta = scale * sigmoid(x) over n elements (use_beta_sigmoid_in_kernel; scale 2 with
 * allow_neg_eigval; reference _compat/kda.py:202-206, FLA fused_beta_sigmoid forward).
 * x fp32 (is_bf16 = 0) or bf16 (1); beta fp32.  The backward is fdr_chunk_bwd's
 * beta_sigmoid argument.
 */
hipError_t fdr_beta_sigmoid_fwd(const void* x, int is_bf16, float scale, float* beta, long long n,
                                hipStream_t stream);

/*
 * Grouped value heads: dq / dk summed over each q / k head's group of value heads.
 * x bf16 [rows, heads, group, K] (the chunk kernels' per-value-head dq or dk, rows = B*T,
 * heads = the q / k heads H, group = HV / H), out bf16 [rows, heads, K]:
 *   out[r, h, :] = bf16(sum_j x[r, h, j, :]), in fp32, j ascending.
 * Replaces the reshape-and-sum over FLA's per-value-head dq / dk (FLA's head map
 * i_h = i_hv // (HV / H); the reference's GVA path, runtime.py:85, leaves it to torch).
 */
hipError_t fdr_group_sum(const void* x, void* out, long long rows, int heads, int group, int K, hipStream_t stream);

/*
 * q / k L2 normalisation over K = 128 (use_qk_l2norm_in_kernel=True, reference
 * _compat/kda.py:202-206; FLA l2norm_fwd / l2norm_bwd), `rows` rows of 128 channels,
 * bf16 (is_bf16 = 1) or fp32:
 *   fwd: rstd = (sum x^2 + eps)^-1/2 (fp32 per row, may be null), y = x rstd
 *   bwd: dx = rstd (dy - y (y . dy)) with y = x rstd
 */
hipError_t fdr_l2norm_fwd(const void* x, int is_bf16, void* y, float* rstd, long long rows, int K, float eps,
                          hipStream_t stream);

hipError_t fdr_l2norm_bwd(const void* x, int is_bf16, const float* rstd, const void* dy, void* dx,
                          long long rows, int K, hipStream_t stream);

/*
 * Affine-step form of the two state recurrences (for small B*H, where the
 * sequential chain and not HBM sets the time).  The same results as
 * fdr_state_bwd / fdr_fwd_h, split into chunk-parallel and sequential parts:
 *
 *   fdr_affine_prep_bwd:  M_c = w_c^T kg_c,  Y_c = scale qg_c^T dO_c - w_c^T dv_c
 *                         (dv_c = Aqk_c^T dO_c written to dv_out, or dv_in given)
 *   fdr_affine_prep_fwd:  N_c = kg_c^T w_c,  Z_c = kg_c^T u_c
 *   fdr_affine_scan:      S <- diag(2^g_last) S - A_c S + Y_c, states[c] = S before step c
 *                         (reverse = 1: c = NT-1 .. 0, the backward dh; 0: the forward h)
 *   fdr_affine_side:      out_c = addend_c + sign * rowfac_t * (x_c states[c])
 *                         (dR = dv + [2^(g_last - g_t)] k dh;  v_new = u - w h)
 *
 * Together they replace the reference's two state recurrences (see fdr_state_bwd
 * and fdr_fwd_h: backends/backward.py:117-121, kernels/vector_state_gpu.py:47-67).
 * `step` (bf16, B*NT*H*K*K elements) and `offset` (fp32, B*NT*H*K*V) are
 * workspaces in this library's private fragment order, written by a prep call and
 * read by a scan call.  Gate conventions as for fdr_state_bwd / fdr_fwd_h (for
 * gate_mode 2, q/k are qg/kg).  A scan or side call takes one or two independent
 * problems (a forward and a backward recurrence run side by side); value_block
 * (16, 32 or 64) is the value-tile width of one scan work-group.
 */
typedef struct fdr_scan_problem {
  const void* step;          /* bf16 workspace from a prep call */
  const float* offset;       /* fp32 workspace from the same prep call */
  const float* g;            /* gate cumsum (log2), null for gate_mode 0 */
  const float* initial;      /* fp32 [B,H,K,V] or null (zero) */
  void* states;              /* bf16 [B,T/64,H,K,V] */
  float* final_state;        /* fp32 [B,H,K,V] or null */
  int gate_mode;
  int reverse;
  int state_v_first;         /* initial / final_state are [B,H,V,K] instead of [B,H,K,V] */
} fdr_scan_problem;

typedef struct fdr_side_problem {
  const void* x;             /* bf16 [B,T,H,K]: kg | k (backward), w (forward) */
  const void* states;        /* bf16 [B,T/64,H,K,V] from fdr_affine_scan */
  const void* addend;        /* bf16 [B,T,H,V]: dv_local (backward), u (forward) */
  const float* row_gate;     /* scalar gate cumsum for the factor 2^(g_last - g_t), or null */
  void* out;                 /* bf16 [B,T,H,V]: dR | v_new */
  float sign;                /* +1 (backward) or -1 (forward) */
} fdr_side_problem;

hipError_t fdr_affine_prep_bwd(const void* q, const void* k, const void* w, const float* g, int gate_mode,
                               const void* dO, const float* aqk, const void* dv_in, void* step,
                               float* offset, void* dv_out, int B, int T, int H, int K, int V, int chunk,
                               float scale, hipStream_t stream);

hipError_t fdr_affine_prep_fwd(const void* k, const void* w, const void* u, const float* g, int gate_mode,
                               void* step, float* offset, int B, int T, int H, int K, int V, int chunk,
                               hipStream_t stream);

/* fdr_affine_prep_bwd and fdr_affine_prep_fwd in one launch (the recompute policy's two
 * recurrences, same gate_mode; k is kg for gate_mode 2, raw k otherwise). */
hipError_t fdr_affine_prep_pair(const void* q, const void* k, const void* w, const void* u, const float* g,
                                int gate_mode, const void* dO, const float* aqk, const void* dv_in,
                                void* step_bwd, float* offset_bwd, void* dv_out, void* step_fwd,
                                float* offset_fwd, int B, int T, int H, int K, int V, int chunk, float scale,
                                hipStream_t stream);

hipError_t fdr_affine_scan(const fdr_scan_problem* problems, int n_problems, int B, int T, int H, int K,
                           int V, int chunk, int value_block, hipStream_t stream);

hipError_t fdr_affine_side(const fdr_side_problem* problems, int n_problems, int B, int T, int H, int K,
                           int V, int chunk, hipStream_t stream);

/*
 * Diagnostics, no counterpart in the reference: plain HBM streaming with 16-byte lanes,
 * the ceiling the path's roofline fractions are read against.  mode 0 reads `bytes` of src
 * (dst receives grid x 16 bytes), 1 writes `bytes` of dst, 2 copies `bytes` src -> dst; `grid`
 * work-groups of 256 threads stride over the buffer.
 */
hipError_t fdr_stream_probe(int mode, const void* src, void* dst, long long bytes, int grid, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* REWY_AMD_H */
