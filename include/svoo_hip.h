/*
 * svoo_hip.h -- C ABI of the MI355X (gfx950) SVOO online sparse-attention hot path.
 *
 * Conventions
 *   - All tensor arguments are device pointers to contiguous row-major arrays owned by the caller.
 *     bf16 data is passed as uint16_t bit patterns.  The library never allocates or frees memory;
 *     entry points that need scratch take (workspace, ws_bytes) sized by the matching
 *     *_workspace_size() query.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Every entry point only
 *     enqueues work on that stream and never synchronises the host.
 *   - Return value: SVOO_OK (0) or a negative SVOO_ERR_* code; svoo_last_error() describes the failure.
 *   - Shapes use the reference's names: BH = batch*heads, N/S = tokens, D = head dim, QC/KC = query/key
 *     cluster counts.
 *   - Head dim: every row of Q, K, V and of the centroids holds 128 elements (256 bytes).  D (1..128) is the
 *     head dim; for D < 128 elements D..127 of every row must be zero (the Python operators pad).  D sets the
 *     score and softmax scale 1/sqrt(D); on zero-padded rows every dot, centroid and label equals that of the
 *     D-element rows.  Outputs are rows of 128 with zeros past D.
 *
 * Reference paths below are relative to the root of the reference repository (Mutual-Luo/SVOO).
 */
#ifndef SVOO_HIP_H_
#define SVOO_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SVOO_OK = 0,
  SVOO_ERR_INVALID_ARG = -1,
  SVOO_ERR_UNSUPPORTED = -2,
  SVOO_ERR_WORKSPACE = -3,
  SVOO_ERR_HIP = -4
};

/* Library version (major*10000 + minor*100 + patch) and last error message of the calling thread. */
int svoo_version(void);
const char* svoo_last_error(void);

/* ---------------------------------------------------------------------------------------------
 * Cluster sort: stable counting sort of labels[BH][N] (values in [0, K)).
 *   sorted_idx[b][s]   original token index at sorted position s (ascending index inside a cluster)
 *   sizes[b][k]        bincount of the labels
 *   offsets[b][k]      exclusive prefix of sizes
 *   sorted_labels      optional (may be NULL): labels[b][sorted_idx[b][s]]
 * Replaces torch.argsort(labels) in svoo/kernels/triton/permute.py:90 and
 * torch.sort(cluster_ids) in svoo/co_clustering.py:273-274 (made stable here).
 * ------------------------------------------------------------------------------------------- */
size_t svoo_cluster_sort_workspace_size(int bh, int n, int k);
int svoo_cluster_sort(const int32_t* labels, int bh, int n, int k, int32_t* sorted_idx, int32_t* sizes,
                      int32_t* offsets, int32_t* sorted_labels, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Row gather / scatter along the token axis (rows of row_bytes bytes, a multiple of 16).
 *   svoo_permute_rows:   y[b][s] = x[b][idx[b][s]],  s < n_out, idx values in [0, n_in)
 *     replaces _permute_kernel / permute_tensor_by_labels_triton, svoo/kernels/triton/permute.py:9-35,68-102
 *     (also the centroid initialisation gather, svoo/co_clustering.py:2417-2421)
 *   svoo_permute_rows2:  the same for two tensors sharing one index (K and V, svoo/models/wan/attention.py:1039-1042)
 *   svoo_unpermute_rows: x[b][idx[b][s]] = y[b][s]
 *     replaces _inverse_permute_kernel / apply_inverse_permutation_triton, svoo/kernels/triton/permute.py:38-65,105-130
 *   svoo_unpermute_rows_bshd: the same scatter into the [B, S, H, D] layout (bh = B*H rows of y), i.e.
 *     apply_inverse_permutation_triton followed by transpose(1, 2).flatten(2, 3) of
 *     svoo/models/wan/attention.py:1211-1215 in one pass
 * ------------------------------------------------------------------------------------------- */
int svoo_permute_rows(const void* x, const int32_t* idx, void* y, int bh, int n_in, int n_out, int row_bytes,
                      void* stream);
int svoo_permute_rows2(const void* x0, const void* x1, const int32_t* idx, void* y0, void* y1, int bh, int n,
                       int row_bytes, void* stream);
int svoo_unpermute_rows(const void* y, const int32_t* idx, void* x, int bh, int n, int row_bytes, void* stream);
int svoo_unpermute_rows_bshd(const void* y, const int32_t* idx, void* x, int bh, int n, int heads, int row_bytes,
                             void* stream);

/* ---------------------------------------------------------------------------------------------
 * Centroid update over cluster-sorted tokens: new_c[b][k] = bf16(f32(sum of members) / f32(size)),
 * sizes[b][k] == 0 keeps old_c[b][k].  Sums are exact (fp64), so the result is order independent.
 * Inputs come from svoo_cluster_sort (sorted_idx, sorted_labels, sizes).  new_c may alias old_c.
 * Replaces triton_centroid_update_sorted_euclid + _centroid_update_chunk_kernel,
 * svoo/co_clustering.py:181-303.
 * ------------------------------------------------------------------------------------------- */
size_t svoo_centroid_update_workspace_size(int bh, int k, int d);
int svoo_centroid_update(const uint16_t* x, const int32_t* sorted_idx, const int32_t* sorted_labels,
                         const int32_t* sizes, const uint16_t* old_c, uint16_t* new_c, int bh, int n, int k, int d,
                         void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Row L2 normalisation to fp32: y = x / sqrt(sum(x^2) + eps); x is bf16 (x_is_bf16=1) or fp32.
 * Replaces triton_l2norm_forward / _l2_norm_fwd_fused, svoo/kernels/triton/l2norm.py:8-80.
 * ------------------------------------------------------------------------------------------- */
int svoo_l2norm_rows(const void* x, int x_is_bf16, float* y, long long rows, int cols, float eps, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Element-type conversion of n contiguous values: types 0 bf16, 1 fp16, 2 fp32; to bf16 / fp16 by rounding to
 * nearest even (through fp32).  The operators take fp16 and fp32 tensors by rounding them to bf16, the type
 * every kernel here computes in, and return results in the caller's type; the reference's Triton kernels load
 * any float input as fp32 (svoo/co_clustering.py:2121, :2197) and FlashInfer takes fp16 or bf16
 * (svoo/utils/flashinfer_sparse.py:117-124).
 * ------------------------------------------------------------------------------------------- */
int svoo_convert(const void* src, int src_type, void* dst, int dst_type, long long n, void* stream);
/* rows[r] of src_cols elements -> rows of dst_cols: the first min(src_cols, dst_cols) converted, the rest zero
 * (the padding of a head dim below 128 and its removal). */
int svoo_convert_rows(const void* src, int src_type, int src_cols, void* dst, int dst_type, int dst_cols,
                      long long rows, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Co-clustering (profile-space k-means).
 *   svoo_cocluster_prep: P = l2norm(bf16(A B^T)) ([BH][J][KP], optional output), E = P B split into
 *     E_hi = bf16(E), E_lo = bf16(E - E_hi), both [BH][jpad][D]; rows J..jpad-1 repeat row J-1.
 *     Replaces torch.matmul + triton_l2norm_forward, svoo/co_clustering.py:2427-2428,2440-2441.
 *   svoo_cocluster_assign: labels[b][n] = argmax_j x[b][n] . (E_hi + E_lo)[b][j]  (first j on ties),
 *     with E_hi / E_lo as svoo_cocluster_prep writes them (padding rows repeating row J-1);
 *     equal to argmin_j 2 - 2 (x C^T / ||x C^T||) . P_j of profile_norm_triton + fused_cocluster_assign_triton,
 *     svoo/co_clustering.py:2086-2400, because ||x C^T|| > 0 is a per-token constant.
 *   svoo_co_cluster: max_iters x (key step, query step), all on device, no host synchronisation.
 *     Replaces co_cluster_tokens, svoo/co_clustering.py:2402-2451.  q_cent / k_cent hold the initial
 *     centroids on entry and the final ones on return; labels, sizes and the stable sort of the final
 *     labels (sorted_idx, offsets) are outputs.
 * ------------------------------------------------------------------------------------------- */
int svoo_cocluster_prep(const uint16_t* a, const uint16_t* b, uint16_t* e_hi, uint16_t* e_lo, float* profile, int bh,
                        int j, int kp, int d, int jpad, void* stream);
int svoo_cocluster_assign(const uint16_t* x, const uint16_t* e_hi, const uint16_t* e_lo, int32_t* labels, int bh,
                          int n, int j, int jpad, int d, void* stream);
size_t svoo_co_cluster_workspace_size(int bh, int n, int qc, int kc, int d);
int svoo_co_cluster(const uint16_t* q, const uint16_t* k, int bh, int n, int d, int qc, int kc, int max_iters,
                    uint16_t* q_cent, uint16_t* k_cent, int32_t* q_labels, int32_t* k_labels, int32_t* q_sizes,
                    int32_t* k_sizes, int32_t* q_sorted_idx, int32_t* k_sorted_idx, int32_t* q_offsets,
                    int32_t* k_offsets, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Scaled centroid scores: scores[bh][i][j] = bf16(bf16(qc_i . kc_j) * f32(1 / sqrt(D))), with
 * bf16(exact dot) as a bf16 matmul output (rounded through fp32); qc [BH][QN][D], kc [BH][KN][D] bf16.
 * Replaces the attn_scores of identify_dynamic_map, svoo/co_clustering.py:578
 * (torch.matmul(query_centroids, key_centroids.transpose(-2, -1)) / D**0.5).
 * ------------------------------------------------------------------------------------------- */
int svoo_centroid_scores(const uint16_t* qc, const uint16_t* kc, int bh, int qn, int kn, int d, uint16_t* scores,
                         void* stream);

/* ---------------------------------------------------------------------------------------------
 * Block mask: per (b, h, q-cluster) row, weighted softmax of the scaled centroid scores, stable
 * descending sort, top-p with per-head minimum keep and optional cap, scattered back to a bool map.
 *   preserve[h], cap[h]: per-head counts computed on the host from min_kc_ratio / max_kc_ratio
 *   (cap 0 = none); p_storage: top_p rounded to the storage dtype; full != 0 gives an all-true map
 *   (qc, kc, k_sizes, preserve, cap and scores may then be NULL).
 *   map[b][h][i][j] (uint8 0/1), lengths[b][h][i] = kept key clusters (may be NULL).
 *   scores: [B*H][QN][KN] bf16 buffer of the caller that receives the scaled centroid scores
 *   (svoo_centroid_scores) from which the mask is built.
 * Replaces weighted_softmax + identify_dynamic_map, svoo/co_clustering.py:544-633.
 * ------------------------------------------------------------------------------------------- */
int svoo_block_mask(const uint16_t* qc, const uint16_t* kc, const int32_t* k_sizes, const int32_t* preserve,
                    const int32_t* cap, int b, int h, int qn, int kn, int d, float p_storage, int full, uint8_t* map,
                    int32_t* lengths, uint16_t* scores, void* stream);

/* Weighted softmax of bf16 scores [rows][cols] with fp32 weights (row stride weight_row_stride, 0 = one
 * row shared by all) -> bf16 probabilities.
 * Replaces weighted_softmax, svoo/co_clustering.py:544-553 (fp64 evaluation, rounded via fp32 to bf16). */
int svoo_weighted_softmax(const uint16_t* scores, const float* weights, long long weight_row_stride,
                          uint16_t* out, long long rows, int cols, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Variable-block-sparse attention over cluster-contiguous tokens.
 *   q, k, v, o: [BH][S][D] bf16; map: [BH][QN][KN] uint8; q_sizes [BH][QN], k_sizes [BH][KN] int32.
 *   For each (b, i): O_i = softmax(Q_i K_S^T / sqrt(D)) V_S over the active key clusters S (ascending),
 *   fp32 online softmax, bf16 MFMA; rows of a query cluster with no active keys are zero.
 *   status (device int32, may be NULL) receives 0, or 1 when the sizes of a head do not sum to S
 *   (every output row of that head is then NaN, so the error is visible without a host read-back).
 *   Limits (SVOO_ERR_UNSUPPORTED beyond them): D = 128, KN <= 4096, ceil(S / 256) + QN < 32768.
 * Replaces dynamic_block_sparse_fwd_flashinfer (svoo/co_clustering.py:1231-1311, with the plan of
 * svoo/utils/flashinfer_sparse.py:43-244) and dynamic_block_sparse_fwd_triton (svoo/co_clustering.py:949-1228).
 *   svoo_vbsa_segments: the per-(b, i) active key segments (start, length), ascending cluster order,
 *   that the attention kernel walks: seg_start/seg_len [BH][QN][KN], seg_count [BH][QN].  Expanding them
 *   gives the reference's kv_indices (svoo/utils/flashinfer_sparse.py:43-97) without the head offset.
 * ------------------------------------------------------------------------------------------- */
size_t svoo_vbsa_workspace_size(int bh, int s, int qn, int kn);
int svoo_vbsa_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* map,
                  const int32_t* q_sizes, const int32_t* k_sizes, uint16_t* o, int bh, int s, int d, int qn, int kn,
                  void* workspace, size_t ws_bytes, int32_t* status, void* stream);
int svoo_vbsa_segments(const uint8_t* map, const int32_t* k_sizes, int bh, int qn, int kn, int32_t* seg_start,
                       int32_t* seg_len, int32_t* seg_count, void* stream);
/* svoo_vbsa_fused_fwd: the same attention on Q, K, V in token order ([BH][S][D], BH = B*H), read through the
 *   clusters' stable sort (q_sorted_idx / k_sorted_idx [BH][S], as svoo_co_cluster returns them), with each
 *   output row written to its token's place in o_bshd [B][S][H][D].  Equal to svoo_permute_rows (Q),
 *   svoo_permute_rows2 (K, V), svoo_vbsa_fwd and svoo_unpermute_rows_bshd in sequence, in one pass.
 *   Replaces the permutes, dynamic_block_sparse_fwd_flashinfer and apply_inverse_permutation_triton +
 *   transpose of svoo/models/wan/attention.py:1037-1042, 1196-1215. */
int svoo_vbsa_fused_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* q_sorted_idx,
                        const int32_t* k_sorted_idx, const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes,
                        uint16_t* o_bshd, int bh, int heads, int s, int d, int qn, int kn, void* workspace,
                        size_t ws_bytes, int32_t* status, void* stream);
/* svoo_vbsa_fused_fwd_noalloc: svoo_vbsa_fused_fwd without a workspace argument; it allocates nothing.
 *   No counterpart in the reference.  It is for callers that cannot allocate device memory per call (code
 *   under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The plan lives in a
 *   static device array of SVOO_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call whose
 *   plan (svoo_vbsa_workspace_size(bh, s, qn, kn)) exceeds it returns SVOO_ERR_WORKSPACE before any launch.
 *   Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other
 *   host threads) race and must be serialised by the caller. */
#define SVOO_NOALLOC_SCRATCH_BYTES (4u << 20)
int svoo_vbsa_fused_fwd_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* q_sorted_idx,
                                const int32_t* k_sorted_idx, const uint8_t* map, const int32_t* q_sizes,
                                const int32_t* k_sizes, uint16_t* o_bshd, int bh, int heads, int s, int d, int qn,
                                int kn, int32_t* status, void* stream);

/* ---------------------------------------------------------------------------------------------
 * EAR (error-aware routing with centroid compensation).  All token inputs are cluster-contiguous
 * (permuted); k_offsets [BH][KN] is the exclusive prefix of k_sizes.
 *   svoo_ear_value_stats: per key cluster j the value centroid v_cent[b][j] (compute_vc != 0:
 *     bf16(bf16(exact member sum) / bf16(max(|K_j|, 1))), an empty cluster gives 0; compute_vc == 0
 *     reads it), vc_sq[b][j] = |v_cent|^2 (fp32) and, with u_t = v_t - v_cent_j, tok_stats[b][t] =
 *     {|u_t|^2, u_t . v_cent_j} (fp32 pairs, [BH][N][2]; the reference keeps |v_t|^2 and v_cent_j . v_t,
 *     from which these follow).  Replaces _compute_value_centroids (svoo/models/wan/attention.py:593-610)
 *     and _precompute_v_stats_kernel (svoo/co_clustering.py:1315-1396).
 *   svoo_ear_centroid_logits: c[b][i][j] = bf16(bf16(qc_i . kc_j) * D^-0.5), exact dot (the same
 *     values as svoo_centroid_scores).
 *     Replaces the einsum of svoo/co_clustering.py:1725.
 *   svoo_ear_efficiency: eff[b][i][j] = log(max(err_ij, eps)) - gamma log(max(|Q_i||K_j|, eps)) with
 *     err_ij = sum_t || e^{a_t} v_t - e^{c_ij} vc_j ||^2 over the tokens of key cluster j,
 *     a_t = qc_i . k_t / sqrt(D) (fp32 MFMA), evaluated with the exponents shifted by
 *     max(c_ij, max_t a_t) and in the centroid-difference form that avoids the cancellation of the
 *     reference's expansion (fp32 [BH][QN][KN]).  Replaces error_estimation_triton +
 *     _error_estimation_kernel, svoo/co_clustering.py:1399-1689.
 *   svoo_ear_select: the EAR block map (uint8 [B][H][QN][KN]) from c and eff: budget = area of the
 *     top-p prefix (at least budget_preserve[h]) of the bf16 softmax of c + bf16(log(|K| + 1e-8)),
 *     stably sorted; the first preserve[h] budget-ordered clusters are kept; the others are taken in
 *     descending efficiency (stable) while the area before them is below the remaining budget.  Areas
 *     are exact int64.  Replaces the selection of identify_dynamic_map_estimated,
 *     svoo/co_clustering.py:1692-1797.
 *   svoo_vbsa_ear_fwd: for each (b, i), softmax attention of Q_i over the tokens of the active key
 *     clusters and the (k_cent_j, v_cent_j) pairs of the inactive ones, scored
 *     q . k_cent_j / sqrt(D) + log(|K_j| + 1e-6): one online softmax (fp32, bf16 MFMA).  Workspace and
 *     status as svoo_vbsa_fwd.  Replaces dynamic_block_sparse_prune_fwd_flashinfer (FlashInfer
 *     attention with return_lse + _fused_qc_kernel_opt), svoo/co_clustering.py:1801-2050.
 * ------------------------------------------------------------------------------------------- */
int svoo_ear_value_stats(const uint16_t* v_perm, const int32_t* k_offsets, const int32_t* k_sizes, int bh, int n,
                         int kn, int d, int compute_vc, uint16_t* v_cent, float* vc_sq, float* tok_stats,
                         void* stream);
int svoo_ear_centroid_logits(const uint16_t* qc, const uint16_t* kc, int bh, int qn, int kn, int d,
                             uint16_t* c_logits, void* stream);
int svoo_ear_efficiency(const uint16_t* qc, const uint16_t* k_perm, const uint16_t* c_logits, const float* tok_stats,
                        const float* vc_sq, const int32_t* q_sizes, const int32_t* k_sizes, const int32_t* k_offsets,
                        int bh, int n, int qn, int kn, int d, float gamma, float eps, float* eff, void* stream);
int svoo_ear_select(const uint16_t* c_logits, const float* eff, const int32_t* q_sizes, const int32_t* k_sizes,
                    const int32_t* preserve, const int32_t* budget_preserve, int b, int h, int qn, int kn,
                    float p_storage, uint8_t* map, void* stream);
int svoo_vbsa_ear_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* k_cent,
                      const uint16_t* v_cent, const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes,
                      uint16_t* o, int bh, int s, int d, int qn, int kn, void* workspace, size_t ws_bytes,
                      int32_t* status, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Offline profile producer: exact attention sparsity.
 *   svoo_exact_sparsity_counts: for each of `rows` rows of n bf16 attention scores, the smallest
 *   number of keys whose softmax weights (of scores * scale) hold `threshold` of the row's mass;
 *   counts int32 [rows].  Weights are float(exp(double(s - max))) with s = float(score) * scale in
 *   fp32; masses are fp64 sums in descending order.  Replaces the sort / cumsum / searchsorted of
 *   _exact_counts_from_scores and counts_from_sorted_probabilities_triton
 *   (svoo/sparsity/exact.py:110-155, svoo/kernels/triton/sparsity.py:9-106).
 * ------------------------------------------------------------------------------------------- */
int svoo_exact_sparsity_counts(const uint16_t* scores, long long rows, int n, float scale, float threshold,
                               int32_t* counts, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Diagnostic (no reference counterpart): runs one v_mfma_f32_32x32x16_bf16 and one
 * v_mfma_f32_16x16x32_bf16 on index-coded operands and writes the raw per-lane accumulators
 * (out32: 64 lanes x 16 floats, out16: 64 lanes x 4 floats), so tests can confirm the operand
 * layouts the kernels assume.
 * ------------------------------------------------------------------------------------------- */
int svoo_probe_mfma_layout(float* out32, float* out16, void* stream);
/* Diagnostic (no reference counterpart): the same for v_mfma_f64_16x16x4_f64 (out: 64 lanes x 4 doubles,
 * D[i][j] = 64 i + j by the assumed operand layout). */
int svoo_probe_mfma_f64_layout(double* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SVOO_HIP_H_ */
