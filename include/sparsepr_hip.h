/*
 * libsparsepr_hip.so — C ABI of the MI355X (gfx950) SparsePR sparse-attention path.
 *
 * Conventions for every entry point:
 *   - pointers are device pointers (HIP), tensors are dense row-major;
 *   - sizes are element counts unless named *_bytes;
 *   - work is enqueued on `stream`; no entry point synchronises the host;
 *   - return value: 0 = ok, 1 = invalid argument, 2 = launch error,
 *     3 = workspace too small; spr_last_error() describes the last failure
 *     on the calling thread;
 *   - dtype codes: 0 = bfloat16, 1 = float16, 2 = float32;
 *   - outputs are written, never allocated: callers own all memory
 *     (torch's caching allocator on the Python side).
 *
 * Each declaration names the reference interface it replaces (file:line in
 * PardisTaghavi/SparsePR).
 */
#ifndef SPARSEPR_HIP_H
#define SPARSEPR_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* spr_last_error(void);
int spr_abi_version(void);

/* ---------------------------------------------------------------- permute
 * src/sparsepr/kernels/triton/permute.py:126-172 permute_tensor_by_labels_triton
 *   dst[b, s, :] = src[b, idx[b, s], :]            (rows of row_bytes bytes) */
int spr_permute_rows(const void* src, const int32_t* idx, void* dst, int64_t bh, int64_t rows,
                     int64_t row_bytes, hipStream_t stream);
/* permute.py:235-274 apply_inverse_permutation_triton
 *   dst[b, idx[b, s], :] = src[b, s, :] */
int spr_inverse_permute_rows(const void* src, const int32_t* idx, void* dst, int64_t bh, int64_t rows,
                             int64_t row_bytes, hipStream_t stream);
/* The same (permute.py:235-274; the adapters pass the video part of the attention output,
 * a slice of a longer tensor, hunyuanvideo.py:229-231) with head b's source rows starting
 * src_head_bytes after head b - 1's (src_head_bytes >= rows * row_bytes): read in place. */
int spr_inverse_permute_rows_strided(const void* src, int64_t src_head_bytes, const int32_t* idx, void* dst,
                                     int64_t bh, int64_t rows, int64_t row_bytes, hipStream_t stream);
/* permute.py:175-232 permute_concatenated_tensors_by_labels_triton
 *   dst[b, s, :] = cat(prefix[b], suffix[b])[idx[b, s], :] */
int spr_permute_concat_rows(const void* prefix, const void* suffix, const int32_t* idx, void* dst, int64_t bh,
                            int64_t prefix_rows, int64_t suffix_rows, int64_t row_bytes, hipStream_t stream);
/* n8_v6.py:1234-1235 / residual_repair.py:330-363 probe-row gathers, kmeans_triton_impl.py:91-96 init gather
 *   dst[b, j, :] = src[b, idx[b, j], :], j < dst_rows */
int spr_gather_rows(const void* src, int64_t src_rows, const int32_t* idx, void* dst, int64_t dst_rows,
                    int64_t bh, int64_t row_bytes, hipStream_t stream);
/* residual_repair.py:257-282 _n8_exact_probe_scatter_kernel
 *   dst[b, idx[b, j], :] = src[b, j, :], j < src_rows */
int spr_scatter_rows(const void* src, int64_t src_rows, const int32_t* idx, void* dst, int64_t dst_rows,
                     int64_t bh, int64_t row_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- label sort
 * torch.argsort(labels) at permute.py:154-157, n8_v6.py:905, hunyuanvideo.py:189,
 * plus torch.sort in centroid_update_triton.py:364 and the cluster sizes of
 * kmeans_utils.py:1110-1121.  Stable: equal labels keep ascending token order.
 *   labels int32 [rows, n] in [0, k) -> sorted_idx int32 [rows, n],
 *   sizes int32 [rows, k] (nullable), offsets int32 [rows, k + 1] (nullable). */
size_t spr_argsort_labels_workspace(int64_t rows, int64_t n, int32_t k);
int spr_argsort_labels(const int32_t* labels, int64_t rows, int64_t n, int32_t k, int32_t* sorted_idx,
                       int32_t* sizes, int32_t* offsets, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* ---------------------------------------------------------------- k-means
 * assign_euclid_triton.py:1282-1283 c_sq = (centroids.float() ** 2).sum(-1) */
int spr_centroid_sq(const void* c, int32_t dtype, int64_t rows, int32_t d, float* c_sq, hipStream_t stream);
/* assign_euclid_triton.py:1238-1412 euclid_assign_triton / kmeans_utils.py:775-893 inline-x_sq variant.
 *   bf16 x [batch, n, d], bf16 centroids [batch, k, d], fp32 c_sq [batch, k];
 *   x_sq fp32 [batch, n] or NULL (computed inline: x_sq_mode 0 = fp32, 1 = bf16 buffer);
 *   x_sq_out fp32 [batch, n] nullable: receives the inline x_sq (when x_sq is NULL) so
 *   later iterations over the same points can pass it back (kmeans_triton_impl.py:84-87
 *   computes it once per Lloyd loop);
 *   labels int32 [batch, n]; d in {64, 128}. */
int spr_kmeans_assign_bf16(const void* x, const void* centroids, const float* c_sq, const float* x_sq,
                           int32_t x_sq_mode, float* x_sq_out, int64_t batch, int64_t n, int32_t k, int32_t d,
                           int32_t* labels, hipStream_t stream);
/* assign_euclid_triton.py:803-1030 / kmeans_utils.py:775-893 on fp32 inputs, where
 * tl.dot rounds both operands to TF32 (nearest, ties away): the role-space k-means of
 * N8V6Core.route (n8_v6.py:719,790).  dist = max((x_sq + c_sq) - 2 tf32(x).tf32(c), 0)
 *   with exact TF32 products summed in fp32, lowest index among exact minima.
 *   x fp32 [batch, n, d], centroids fp32 [batch, k, d], c_sq fp32 [batch, k];
 *   x_sq fp32 [batch, n] or NULL (inline: fp32 sum of the fp32 squares of x);
 *   x_sq_out nullable as for spr_kmeans_assign_bf16; d a multiple of 16 up to 128. */
int spr_kmeans_assign_tf32(const float* x, const float* centroids, const float* c_sq, const float* x_sq,
                           float* x_sq_out, int64_t batch, int64_t n, int32_t k, int32_t d, int32_t* labels,
                           hipStream_t stream);
/* centroid_update_triton.py:316-386 triton_centroid_update_sorted_euclid,
 * centroid_reduction.py:138-196 original_centroids_triton, n8_ops.cu:255-269 finalize.
 *   Means of the rows of each cluster (sorted_idx/offsets from spr_argsort_labels), fp64
 *   accumulation, empty clusters keep `old`.  dtype 0 (bf16, d in {64,128}) or 2 (fp32,
 *   d a multiple of 16 up to 128).  Nullable outputs: mean32 fp32 [batch,k,d], out dtype [batch,k,d],
 *   shift_max fp32 scalar (pre-zeroed; max_k ||out-old||), sums_accum fp32 += sums,
 *   counts_accum int32 += counts, c_sq_out fp32 [batch,k] = squared norms of `out` (as
 *   spr_centroid_sq computes them, for the next assignment).  Each cluster's rows are split
 *   into slices of 512 (a plan made on the device from the offsets); their fp64 partial sums
 *   go to the workspace (spr_centroid_mean_workspace bytes, with the plan) and are added in
 *   slice order. */
size_t spr_centroid_mean_workspace(int64_t batch, int64_t n, int32_t k, int32_t d);
int spr_centroid_mean(const void* x, int32_t dtype, const int32_t* sorted_idx, const int32_t* offsets,
                      const void* old, int64_t batch, int64_t n, int32_t k, int32_t d, float* mean32, void* out,
                      float* shift_max, float* sums_accum, int32_t* counts_accum, float* c_sq_out,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);
/* operator_kmeans.py:609-679 original_centroids / joint_original_centroids, centroid_reduction.py:
 * 138-196 original_centroids_triton / joint_original_centroids_triton: fp32 means of the rows of
 * x (and of y, nullable, in the same traversal of the sorted index) per cluster, fp64 sums;
 * an empty cluster takes its fp32 fallback row (x_fallback / y_fallback nullable: zeros).
 *   x, y dtype 0 bf16 (d in {64, 128}) or 2 fp32 (d in {16, 32, 48, 64, 128}) [batch, n, d];
 *   sorted_idx / offsets from spr_argsort_labels; x_out, y_out fp32 [batch, k, d];
 *   workspace spr_original_centroids_workspace bytes (0 when no cluster is split). */
size_t spr_original_centroids_workspace(int64_t batch, int64_t n, int32_t k, int32_t d);
int spr_original_centroids(const void* x, const void* y, int32_t dtype, const int32_t* sorted_idx,
                           const int32_t* offsets, int64_t batch, int64_t n, int32_t k, int32_t d,
                           const float* x_fallback, const float* y_fallback, float* x_out, float* y_out,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);
/* n8_ops.cu:198-253 role_cluster_assign_accumulate_q64_kernel (assignment part):
 *   exact FP32 distance (sequential fmaf), lowest index on ties; d in {16,32,48,64}.
 *   best_dist nullable. */
int spr_role_assign_fp32(const float* features, const float* centroids, int64_t batch, int64_t n, int32_t k,
                         int32_t d, int32_t* labels, float* best_dist, hipStream_t stream);

/* ---------------------------------------------------------------- cluster-pair selection
 * kmeans_utils.py:1710-1742 identify_dynamic_map (+ weighted_softmax :1698-1707),
 * n8_v6.py:181-230 _svg_top_p_key_budgets.  One workgroup per (head, q-cluster) row:
 *   s = fl(qc . kc) / sqrt_d (sequential fp32 dot), p = k_size * exp(s - max) / sum,
 *   descending sort (index tie-break), sequential cumsum, keep ranks whose preceding
 *   cumsum <= p (rank 0 always), then the min_kc_ratio floor (`preserve` ranks).
 *   qc fp32 [bh, qn, d], kc fp32 [bh, kn, d], k_sizes int32 [bh, kn] -> map uint8
 *   [bh, qn, kn] (nullable) and budgets int32 [bh, qn] (nullable; the sum of the kept
 *   clusters' sizes, the key-token budgets of n8_v6.py:181-230, whose keep rule is the
 *   same); at least one of the two.  score_bf16 = 1 rounds every intermediate the way
 *   bf16 tensors do in torch (matmul output, scaled score, probabilities, cumsum);
 *   kn <= 4096. */
int spr_topp_map(const float* qc, const float* kc, const int32_t* k_sizes, int64_t bh, int32_t qn, int32_t kn,
                 int32_t d, float sqrt_d, float p, int32_t preserve, int32_t score_bf16, uint8_t* map,
                 int32_t* budgets, hipStream_t stream);
/* n8_ops.cu:271-322,541-571 svg_ear_select_budget (mode 0) and the Triton / CPU selectors
 * selector_budget.py:131-171, n8_v6.py:1088-1111 (mode 1: crossing at sorted position
 * `count`); n8_ops.cu:573-638 svg_ear_select_budget_schedule when ids/counts are given.
 *   scores fp32 [bh, qn, kn], sizes int32 [bh, kn], budgets int32 [bh, qn] ->
 *   out uint8 [bh, qn + 1, kn + 1] (header row/column set as the reference);
 *   ids int32 [bh, qn, kn] + counts int32 [bh, qn] (both or neither). */
int spr_select_budget(const float* scores, const int32_t* sizes, const int32_t* budgets, int64_t bh, int32_t qn,
                      int32_t kn, int32_t mode, uint8_t* out, int32_t* ids, int32_t* counts, hipStream_t stream);
/* n8_ops.cu:324-355,609-638 compact_selected_clusters: ascending kept ids per mask row;
 * entries past counts[row] are left unwritten (the reference returns them uninitialised).
 *   mask uint8 [rows, kn] -> ids int32 [rows, kn], counts int32 [rows]. */
int spr_compact_selected(const uint8_t* mask, int64_t rows, int32_t kn, int32_t* ids, int32_t* counts,
                         hipStream_t stream);
/* kmeans_utils.py:285-303 density_calculation:
 *   out[h] = sum_ij map[h,i,j] qs[h,i] ks[h,j] / (sum_i qs[h,i] * sum_j ks[h,j]). */
int spr_density(const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes, int64_t heads, int32_t qn,
                int32_t kn, float* out, hipStream_t stream);

/* ---------------------------------------------------------------- block-sparse attention
 * kmeans_utils.py:2164-2350 dynamic_block_sparse_fwd_flashinfer (FlashInfer
 * VariableBlockSparseAttentionWrapper.plan / .run), semantics of
 * dynamic_block_sparse_fwd_torch kmeans_utils.py:1748-1841.
 * Plan: per kv head, cluster offsets, 128- and 256-row query tiles and, per q-cluster,
 * the kept non-empty key ranges; the 256-row tiles of a head in decreasing q-cluster key
 * count; after the heads, the order in which the kv heads fill the tile grid (balanced
 * over the 8 XCDs by work).  map uint8 [bh_kv, qn, kn], q_sizes int32 [bh_kv, qn],
 * k_sizes int32 [bh_kv, kn]; sizes are clamped to the s rows; qn <= 4096, kn <= 16384.
 * The plan ends with a header (bh_kv, qn, kn, s) written after the rest of the plan; the
 * run checks plan_bytes on the host, and its kernels compare the header with their own
 * sizes and leave `out` unwritten when it does not match (a plan built for other sizes). */
size_t spr_block_sparse_attention_workspace(int64_t bh_kv, int32_t qn, int32_t kn);
int spr_block_sparse_attention_plan(const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_kv,
                                    int64_t s, int32_t qn, int32_t kn, void* plan, size_t plan_bytes,
                                    hipStream_t stream);
/* n8_ops.cu:573-638 svg_ear_select_budget_schedule / compact_selected_clusters as the
 * attention's work list: the same plan built from a selector schedule instead of the map.
 * ids int32 [bh_kv, qn, kn]: row r's first counts[r] entries are its kept k-clusters in
 * strictly ascending order (as spr_select_budget and spr_compact_selected write them);
 * counts int32 [bh_kv, qn].  An entry outside [0, kn) or not above every earlier entry
 * of its row is ignored, so the plan never lists a key range twice. */
int spr_block_sparse_attention_plan_schedule(const int32_t* ids, const int32_t* counts, const int32_t* q_sizes,
                                             const int32_t* k_sizes, int64_t bh_kv, int64_t s, int32_t qn,
                                             int32_t kn, void* plan, size_t plan_bytes, hipStream_t stream);
/* q bf16 [bh_q, s, d], k/v bf16 [bh_kv, s, d] in cluster-contiguous order; bh_q a
 * multiple of bh_kv (query head h uses kv head h / (bh_q / bh_kv)); d in {64, 128}.
 * out bf16 [bh_q, s, d]: softmax over the kept keys of the row's q-cluster (scale
 * applied to q.k); rows of empty q-clusters are 0.  lse fp32 [bh_q, s] (nullable,
 * natural log of the scaled sum, -inf for an empty row).  q_index int32 [bh_q, s] (nullable):
 * q, out and lse stay in token order and cluster-sorted row r is token q_index[r], which fuses
 * permute_tensor_by_labels_triton of Q and apply_inverse_permutation_triton of the output
 * (hunyuanvideo.py:189-231) into the attention.  k_index int32 [bh_kv, s] (nullable): k and v stay
 * in token order and cluster-sorted key position p is token k_index[p] (the K/V permutation of
 * n8_v6.py:905-925 fused into the key gather). */
int spr_block_sparse_attention_run(const void* q, const void* k, const void* v, const void* plan, size_t plan_bytes,
                                   int64_t bh_q, int64_t bh_kv, int64_t s, int32_t d, int32_t qn, int32_t kn,
                                   float scale, const int32_t* q_index, const int32_t* k_index, void* out, float* lse,
                                   hipStream_t stream);
/* Plan + run in one call; workspace = plan buffer of spr_block_sparse_attention_workspace bytes. */
int spr_block_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* map,
                               const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q, int64_t bh_kv, int64_t s,
                               int32_t d, int32_t qn, int32_t kn, float scale, const int32_t* q_index,
                               const int32_t* k_index, void* out, float* lse, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);
/* spr_block_sparse_attention_run / spr_block_sparse_attention for every element type and
 * head dim the reference's attention takes (kmeans_utils.py:1847-2161 Triton: d in
 * {16, 32, 64, 128}; FlashInfer, kmeans_utils.py:2164-2350: bf16 or fp16): q, k, v and out of
 * dtype 0 bf16 / 1 fp16 (the probabilities P are rounded to the same type); d in
 * {16, 32, 64, 128}.  The calls above are dtype 0. */
int spr_block_sparse_attention_run_ex(const void* q, const void* k, const void* v, const void* plan,
                                      size_t plan_bytes, int64_t bh_q, int64_t bh_kv, int64_t s, int32_t d, int32_t qn,
                                      int32_t kn, float scale, int32_t dtype, const int32_t* q_index,
                                      const int32_t* k_index, void* out, float* lse, hipStream_t stream);
int spr_block_sparse_attention_ex(const void* q, const void* k, const void* v, const uint8_t* map,
                                  const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q, int64_t bh_kv,
                                  int64_t s, int32_t d, int32_t qn, int32_t kn, float scale, int32_t dtype,
                                  const int32_t* q_index, const int32_t* k_index, void* out, float* lse,
                                  void* workspace, size_t workspace_bytes, hipStream_t stream);
/* No counterpart in the reference: spr_block_sparse_attention for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  Same arguments and results, with the plan kept in a fixed 64 MiB device
 * array of the library (one per device, held until the process ends) instead of a
 * workspace; calls no hipMalloc/hipFree.  Returns 3 when the plan for (bh_kv, qn, kn)
 * needs more than 64 MiB (spr_block_sparse_attention_workspace bytes).  Calls that
 * overlap on one device share the array and race; the calling thread's current device
 * must be the stream's device. */
int spr_block_sparse_attention_noalloc(const void* q, const void* k, const void* v, const uint8_t* map,
                                       const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q, int64_t bh_kv,
                                       int64_t s, int32_t d, int32_t qn, int32_t kn, float scale,
                                       const int32_t* q_index, const int32_t* k_index, void* out, float* lse,
                                       hipStream_t stream);
/* n8_v6.py:1236-1243 dense probe attention (F.scaled_dot_product_attention of the probe
 * rows against every key).  q bf16 [bh_q, m, d], k/v bf16 [bh_kv, s_kv, d]; keys split
 * into nsplit ranges computed in parallel and merged; out [bh_q, m, d] (out_dtype 0 =
 * bf16, 2 = fp32); lse fp32 [bh_q, m] nullable. */
size_t spr_dense_attention_workspace(int64_t bh_q, int64_t m, int32_t d, int32_t nsplit);
int spr_dense_attention(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv, int64_t m,
                        int64_t s_kv, int32_t d, float scale, int32_t nsplit, void* out, int32_t out_dtype,
                        float* lse, void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same call site (n8_v6.py:1236-1243, whose keys are the video keys plus the prompt
 * tokens, a slice of the full K/V): kv head h's s_kv rows start kv_head_stride elements
 * after head h - 1's (kv_head_stride >= s_kv * d), so the slice is read in place. */
int spr_dense_attention_strided(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv, int64_t m,
                                int64_t s_kv, int64_t kv_head_stride, int32_t d, float scale, int32_t nsplit,
                                void* out, int32_t out_dtype, float* lse, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);
/* spr_dense_attention_strided with q, k, v of dtype 0 bf16 / 1 fp16, d in {16, 32, 64, 128}
 * and out_dtype 0 bf16, 1 fp16 or 2 fp32 (F.scaled_dot_product_attention takes either
 * half type). */
int spr_dense_attention_strided_ex(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv,
                                   int64_t m, int64_t s_kv, int64_t kv_head_stride, int32_t d, float scale,
                                   int32_t dtype, int32_t nsplit, void* out, int32_t out_dtype, float* lse,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- N8 residual repair
 * residual_repair.py:36-118 select_role_equal_probes(_vectorized), group distances:
 *   dist[b, i] = sum_r (features[b, i, r] - centers[b, labels[b, i], r])^2 in fp32, each
 *   term a separate subtract, multiply and add; the terms are summed sequentially within
 *   groups of 8 consecutive dimensions, then the group sums by a pairwise tree (zero
 *   padded to a power of two), a fixed order, so exact ties reproduce.  features dtype
 *   0 bf16 / 2 fp32; centers fp32 [bh, groups, r]; dist fp32 [bh, n]. */
int spr_probe_distances(const void* features, int32_t dtype, const int32_t* labels, const float* centers, int64_t bh,
                        int64_t n, int32_t groups, int32_t r, float* dist, hipStream_t stream);
/* residual_repair.py:121-260 probe choice.  mode 0 = vectorized (one nearest token per
 * group, largest groups first), 1 = rounds (select_role_equal_probes, more rows than
 * groups), 2 = select_first_token_largest_groups.  rows int32 [bh, count], weights fp32
 * [bh, count] (size / sampled, normalised to mean 1), filled int32 [bh] nullable.
 * groups <= 2048.  workspace (spr_probe_select_workspace bytes, nullable) splits the pass
 * over the tokens across many workgroups per head in modes 0 and 2. */
size_t spr_probe_select_workspace(int64_t bh, int32_t groups);
int spr_probe_select(const float* dist, const int32_t* labels, const int32_t* sizes, int64_t bh, int64_t n,
                     int32_t groups, int32_t count, int32_t mode, int32_t* rows, float* weights, int32_t* filled,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);
/* residual_repair.py:798-857 n8_prepare_output_repair_fit_triton:
 *   x_fit = base[rows], dense_f = float(dense), y_fit = dense_f - x_fit (fp32 [bh, m, d]). */
int spr_repair_fit_prep(const void* base, int32_t base_dtype, const void* dense, int32_t dense_dtype,
                        const int32_t* rows, int64_t bh, int64_t n, int32_t m, int32_t d, float* x_fit,
                        float* dense_f, float* y_fit, hipStream_t stream);
/* residual_repair.py:478-562 n8_repair_apply_output_triton:
 *   out = base + alpha * (((base - x_mean) / x_scale) . left . basis^T + y_mean), the
 *   correction's row norm capped at norm_cap when norm_cap > 0.  base/out bf16
 *   [bh, n, d]; x_mean, x_scale, y_mean fp32 [bh, d]; left, basis fp32 [bh, d, rank];
 *   d in {64, 128}, rank in {16, 32, 64}. */
int spr_repair_apply(const void* base, const float* x_mean, const float* x_scale, const float* y_mean,
                     const float* left, const float* basis, int64_t bh, int64_t n, int32_t d, int32_t rank,
                     float alpha, float norm_cap, void* out, hipStream_t stream);
/* residual_repair.py:737-797 n8_prepare_repair_fit_triton (repair_features "output_role"):
 *   x_fit fp32 [bh, m, d + role_dim] = [base[rows], role[rows]] with role fp32
 *   [bh, n, role_dim]; dense_f, y_fit as spr_repair_fit_prep (role_dim 0 is that call). */
int spr_repair_fit_prep_role(const void* base, int32_t base_dtype, const float* role, int32_t role_dim,
                             const void* dense, int32_t dense_dtype, const int32_t* rows, int64_t bh, int64_t n,
                             int32_t m, int32_t d, float* x_fit, float* dense_f, float* y_fit, hipStream_t stream);
/* residual_repair.py:388-475 n8_repair_apply_triton (kernel :10-92):
 *   out = base + alpha * ((([base, role] - x_mean) / x_scale) . left . basis^T + y_mean), the
 *   correction's row norm capped at norm_cap times the base row's norm when norm_cap > 0.
 *   role fp32 [bh, n, role_dim], role_dim in {0, 16, 32, 48, 64} (0: spr_repair_apply);
 *   x_mean, x_scale fp32 [bh, d + role_dim]; y_mean fp32 [bh, d]; left fp32
 *   [bh, d + role_dim, rank]; basis fp32 [bh, d, rank]; d in {64, 128}, rank in {16, 32, 64}. */
int spr_repair_apply_role(const void* base, const float* role, int32_t role_dim, const float* x_mean,
                          const float* x_scale, const float* y_mean, const float* left, const float* basis,
                          int64_t bh, int64_t n, int32_t d, int32_t rank, float alpha, float norm_cap, void* out,
                          hipStream_t stream);
/* ---- model-edge fusions (spr_qkv.hip) */
/* n8_ops.cu:16-105 wan_qkv_norm_rope_layout_kernel (host :356-413): q, k, v [batch, tokens,
 * channels = heads * head_dim] of dtype (0 bf16, 1 fp16, 2 fp32); RMSNorm over all channels of
 * a token with weights [channels] of the same dtype, rounded to the dtype, then complex-pair
 * RoPE by freq_real / freq_imag fp32 [tokens, head_dim / 2]; outputs [batch, heads, tokens,
 * head_dim] (V relaid out).  head_dim even; 16-byte aligned device pointers. */
int spr_wan_qkv_norm_rope_layout(const void* q, const void* k, const void* v, const void* q_weight,
                                 const void* k_weight, const float* freq_real, const float* freq_imag, int32_t dtype,
                                 int64_t batch, int64_t tokens, int32_t channels, int32_t heads, float epsilon,
                                 void* q_out, void* k_out, void* v_out, hipStream_t stream);
/* n8_ops.cu:107-187 cosmos25_qkv_norm_rope_bshd_kernel (host :415-497): q, k, v [batch, tokens,
 * heads * head_dim] of dtype; RMSNorm over each head's head_dim values with fp32 weights
 * [head_dim], rounded to the dtype, then rotate-half RoPE by fp32 angles [tokens, head_dim]
 * (sincosf); outputs [batch, tokens, heads, head_dim].  head_dim even, epsilon > 0. */
int spr_cosmos25_qkv_norm_rope_bshd(const void* q, const void* k, const void* v, const float* q_weight,
                                    const float* k_weight, const float* rope_angles, int32_t dtype, int64_t batch,
                                    int64_t tokens, int32_t heads, int32_t head_dim, float epsilon, void* q_out,
                                    void* k_out, void* v_out, hipStream_t stream);

/* residual_repair.py:263-465 fit_reduced_rank_residual with basis_source "raw_residual":
 * spr_rrr_fit_ex (below) with basis_source 0.  workspace: spr_rrr_fit_workspace(bh) bytes. */
size_t spr_rrr_fit_workspace(int64_t bh);
int spr_rrr_fit(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p, int32_t d,
                int32_t rank, float ridge, float* x_mean, float* x_scale, float* y_mean, float* left, float* basis,
                void* workspace, size_t workspace_bytes, hipStream_t stream);
/* residual_repair.py:656-700 n8_exact_probe_scatter_triton: out[b, rows[b, j]] =
 * dense[b, j] (rounded to bf16); dense dtype 0 bf16 / 2 fp32; rows outside [0, n) skipped. */
int spr_probe_scatter(const void* dense, int32_t dense_dtype, const int32_t* rows, int64_t bh, int64_t n, int32_t m,
                      int32_t d, void* out, hipStream_t stream);

/* ---------------------------------------------------------------- role projection
 * role_projection.py:16-103 role_projection_rms_triton: out = p / sqrt(max(mean_r p_r^2,
 * 1e-12)), p = x . F~ with F~ the factor rounded to TF32 (nearest, ties away).
 *   x bf16 [bh, n, d], d in {64, 128}; factor fp32 [bh, d, rank], 1 <= rank <= 128 ->
 *   out fp32 [bh, n, rank]. */
int spr_role_projection_rms(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d, int32_t rank,
                            float* out, hipStream_t stream);
/* n8_v6.py:141-149 _role_k_projection_normalize_fp32 (torch.compile'd): p = x . F~ as
 * above, key_scale[h] = max(sqrt(mean over tokens and rank of p^2), 1e-8), out = p / key_scale.
 *   x bf16 [bh, n, d], d in {64, 128}; factor fp32 [bh, d, rank], rank <= 128 -> out fp32
 *   [bh, n, rank], key_scale fp32 [bh].  The per-head sum of p^2 is formed deterministically
 *   (fp64 per-workgroup partials in the workspace, summed in order);
 *   workspace: spr_role_k_projection_workspace(bh, n) bytes. */
size_t spr_role_k_projection_workspace(int64_t bh, int64_t n);
int spr_role_k_projection(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d, int32_t rank,
                          float* out, float* key_scale, void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same under role_kv_matmul_precision (n8_v6.py:77-86,141-178): precision 0 "high" (TF32
 * factor), 1 "highest" (fp32 factor, also compile_role_kv_projection=False's
 * normalize_feature_scale(project_tokens(...)), operator_kmeans.py:540-550), 2 "medium" (bf16
 * factor); out[t][out_col + c] (rows of out_ld floats) = (weight p) / key_scale, so the K and
 * the weighted V features of _role_kv_projection_normalize_fp32 (n8_v6.py:91-103) fill one
 * [bh, n, R_k + R_v] tensor side by side. */
int spr_role_k_projection_ex(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d, int32_t rank,
                             int32_t precision, float weight, float* out, int32_t out_ld, int32_t out_col,
                             float* key_scale, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- SVG-EAR routing scores
 * svg_ear.py:95-192,453-531 svg_ear_value_error_scores_triton (mode 0; Jensen term when
 * jensen_var_cap > 0, var_k_diag [kv_heads, kn, d] fp32), svg_ear.py:195-286,534-600 the
 * grouped variant (same scores), svg_ear.py:7-92,372-450 attention_mass_scores_triton
 * (mode 1; v_sorted, k_centroids, v_centroids, var_k_diag unused).
 *   q_centroids fp32 [q_heads, qn, d]; k_sorted, v_sorted bf16 [kv_heads, t_stored, d]
 *   (tokens in cluster order); k_centroids, v_centroids fp32 [kv_heads, kn, d];
 *   k_sizes int32 [kv_heads, kn] (the clusters' consecutive token runs from token 0;
 *   negative sizes count as 0, runs are clamped to t_stored) -> scores fp32
 *   [q_heads, qn, kn], -inf for an empty cluster.  q_heads = kv_heads * group, d = 128.
 *   Token logits use q rounded to TF32 (nearest, ties away), as tl.dot(input_precision
 *   "tf32") does; the centroid logit uses q in fp32.
 * spr_svg_ear_scores_flops: algorithmic flops of the token logits, 2 q_heads qn tokens d. */
size_t spr_svg_ear_scores_flops(int64_t q_heads, int32_t qn, int64_t tokens);
int spr_svg_ear_scores(const float* q_centroids, const uint16_t* k_sorted, const uint16_t* v_sorted,
                       const float* k_centroids, const float* v_centroids, const float* var_k_diag,
                       float jensen_var_cap, const int32_t* k_sizes, int64_t q_heads, int32_t qn, int32_t kn,
                       int64_t kv_heads, int64_t t_stored, int32_t d, int32_t group, int32_t mode, float* scores,
                       hipStream_t stream);
/* svg_ear.py:289-369 (+ wrapper :603-678) svg_ear_compensation_triton: the sparse output
 * (numerator sparse, denominator 1, running max lse) extended, in blocks of block_k (16 or 32)
 * key clusters, by e^(l_c - M) times the V centroid of every valid (count > 0) cluster the
 * map does not select (reformulation 0 "skipped"), or of every valid cluster minus the
 * selected ones (1 "n3_residual"); l_c = (tf32(q) . tf32(kc_c)) / sqrt(128) + log(max(count_c,
 * 1)), the weights TF32-rounded as the reference's dot products see them.
 * q [bh, tokens, 128] (q_dtype 0 bf16 / 2 fp32), sparse [bh, tokens, 128] (sparse_dtype 0 / 2),
 * lse fp32 [bh, tokens], qlabels int32 [bh, tokens], dmap uint8 [bh, qc1, kn + 1] (row qlabel
 * + 1, column cluster + 1), kcentroids / vcentroids fp32 [bh, kn, 128], kcounts fp32 [bh, kn]
 * -> out fp32 [bh, tokens, 128] = acc / max(denom, 1e-30). */
int spr_svg_ear_compensation(const void* q, int32_t q_dtype, const void* sparse, int32_t sparse_dtype,
                             const float* lse, const int32_t* qlabels, const uint8_t* dmap, int32_t qc1,
                             const float* kcentroids, const float* kcounts, const float* vcentroids, int64_t bh,
                             int64_t tokens, int32_t d, int32_t kn, int32_t reformulation, int32_t block_k,
                             float* out, hipStream_t stream);

/* ---------------------------------------------------------------- N8 role metrics and factors
 * operator_kmeans.py:62-92,491-498 covariance / key_metric_from_queries /
 * value_metric_from_values (rows = deterministic_token_sample positions, :52-59) and
 * :517-531 query_metric_from_key_centroids (sizes = cluster sizes, post_scale = 1 / d):
 *   out fp32 [bh, d, d] = post_scale / max(used, 1) * sum over the used rows (x - mean)(x - mean)^T;
 *   x dtype 0 bf16 / 2 fp32 [bh, n, d], d <= 128; rows int32 [count] shared by the heads
 *   (nullable: all n rows); sizes int32 [bh, n] (nullable, only without rows): a row is used
 *   only when its size is > 0; center = 1 subtracts the used rows' mean. */
int spr_role_metric(const void* x, int32_t dtype, int64_t bh, int64_t n, int32_t d, const int32_t* rows,
                    int32_t count, const int32_t* sizes, int32_t center, float post_scale, float* out,
                    hipStream_t stream);
/* residual_repair.py:263-465 fit_reduced_rank_residual / _fit_reduced_rank_residual_fp32 for
 * every configuration it accepts with m, d <= 128, p <= 128 (or, in the dual form, m < p <= 256
 * with 64 ceil(p / 64) (m | 1) <= 16512: the role-feature fit's p = d + role rank) and
 * rank <= 64:
 *   weighted standardisation (:364-384; weights == NULL: plain mean and unbiased std);
 *   primal ridge solve for m >= p (:424-434), dual for m < p (:386-423, both fit_backend
 *   forms); the top-rank eigenvectors of the weighted output gram of the raw residual
 *   (basis_source 0) or of the fitted values (1) (:435-462; the "full" and "skinny" with
 *   eigh / SVD routes span this subspace); left = weight . basis or x_w^T dual basis
 *   (:463-464).
 *   x [bh, m, p], y [bh, m, d], weights [bh, m] fp32; outputs x_mean [bh, p], x_scale
 *   [bh, p], y_mean [bh, d], left [bh, p, rank], basis [bh, d, rank] (basis columns in
 *   ascending eigenvalue order).  1 <= rank <= min(64, d, m).
 *   workspace: spr_rrr_fit_workspace(bh) bytes of device memory. */
int spr_rrr_fit_ex(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p, int32_t d,
                   int32_t rank, float ridge, int32_t basis_source, float* x_mean, float* x_scale, float* y_mean,
                   float* left, float* basis, void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same fit with the "skinny" route and decomposition_backend "triton_top16"
 * (residual_repair.py:435-451,497-503; the reference's GPU N8 repair, n8_v6.py:1310-1320):
 * the basis is spr_rrr_top16_basis of the weighted raw residual (basis_source 0) or of the
 * weighted fitted values (1).  m = 64, d = 128, rank = 16; p <= 256. */
int spr_rrr_fit_top16(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p,
                      int32_t d, int32_t rank, float ridge, int32_t basis_source, float* x_mean, float* x_scale,
                      float* y_mean, float* left, float* basis, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);
/* rrr_eigensolver.py:86-128 top16_right_basis_triton: values fp32 [bh, 64, 128] -> basis fp32
 * [bh, 128, 16].  A = V V^T; from the QR factor Q0 of the cosine seed C[i][j] =
 * cos((i + 1/2)(j + 1) pi / 64), power_iters steps Q = Y X / sqrt(s) with Y = A Q and (X, s)
 * the inv_sqrt_iters-step Newton-Schulz inverse square root of Y^T Y (s its Frobenius norm);
 * then V^T Q orthonormalised the same way.  An approximation of the top-16 right singular
 * subspace, not the exact one.  The fit uses the reference's defaults, 8 and 6; both counts
 * in [1, 4096]. */
int spr_rrr_top16_basis(const float* values, int64_t bh, int32_t power_iters, int32_t inv_sqrt_iters, float* basis,
                        hipStream_t stream);
/* residual_repair.py:468-506 reduced_rank_output_basis: the top-rank right singular basis of
 * a [bh, m, d] fp32 as the eigenvectors of a^T a (ascending), m, d <= 128, rank <= min(64, d).
 * workspace: spr_rrr_fit_workspace(bh) bytes. */
int spr_rrr_output_basis(const float* a, int64_t bh, int32_t m, int32_t d, int32_t rank, float* basis,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);
/* residual_repair.py:509-587 recover_nonfinite_rrr_state: per head, a non-finite value in any
 * of the five state tensors selects the previous state (prev_* all given) or the zero
 * correction (x_mean 0, x_scale 1, y_mean 0, left 0, basis 0; prev_* all NULL).  out_* may
 * alias the current state; recovered u8 [bh] (nullable). */
int spr_rrr_recover(const float* x_mean, const float* x_scale, const float* y_mean, const float* left,
                    const float* basis, const float* prev_x_mean, const float* prev_x_scale, const float* prev_y_mean,
                    const float* prev_left, const float* prev_basis, int64_t bh, int32_t p, int32_t d, int32_t rank,
                    float* out_x_mean, float* out_x_scale, float* out_y_mean, float* out_left, float* out_basis,
                    uint8_t* recovered, hipStream_t stream);
/* torch.linalg.eigh for the top eigenpairs (operator_kmeans.py:115-118, residual_repair.py:468-506):
 *   mats fp32 [bh, n, n] symmetric (symmetrize = 1: 0.5 (A + A^T)); vecs fp32 [bh, n, rank] the
 *   eigenvectors of the rank largest eigenvalues in ascending order; vals fp32 [bh, rank]
 *   (nullable) their Rayleigh quotients, ascending.  n <= 128, rank <= min(64, n).
 *   Householder tridiagonalisation, multisection on Sturm counts, inverse iteration, Cholesky-QR. */
int spr_sym_top_eig(const float* mats, int64_t bh, int32_t n, int32_t rank, int32_t symmetrize, float* vecs,
                    float* vals, hipStream_t stream);
/* operator_kmeans.py:95-151 metric_factor: factor fp32 [bh, n, rank] = top-rank eigenvectors of
 * 0.5 (M + M^T), column c scaled by sqrt(max(lambda_c, 0) / max(mean max(lambda, 0), 1e-12));
 * workspace spr_metric_factor_workspace(bh, rank) bytes (the eigenvalues). */
size_t spr_metric_factor_workspace(int64_t bh, int32_t rank);
int spr_metric_factor(const float* metric, int64_t bh, int32_t n, int32_t rank, float* factor, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);
/* operator_kmeans.py:219-477 warm_subspace_metric_factor (+ n8_v6.py:478-519 _updated_factor's
 * per-head recovery when prev_factor is given): metric fp32 [bh, n, n], prev_state fp32
 * [bh, n, rank] (the previous basis), prev_factor fp32 [bh, n, rank] (nullable) -> factor,
 * state fp32 [bh, n, rank], recovered uint8 [bh] (nullable).  ortho 0 each_cholesky_qr,
 * 1 each_cholesky_qr2, 2 cholesky_qr, 3 each_qr, 4 final_qr (Householder QR, LAPACK's sign
 * convention as torch.linalg.qr); ritz 0 rayleigh_cholesky, 1 diagonal, 2 previous_scale,
 * 3 full (eigh of the Rayleigh matrix; columns in ascending eigenvalue order, signs are the
 * eigensolver's).  n <= 128, rank <= 64.  The full finish needs
 * spr_warm_metric_factor_workspace(bh, n, rank, ritz) bytes of workspace (0 for the others);
 * spr_warm_metric_factor is the workspace-free form (ritz 0..2). */
size_t spr_warm_metric_factor_workspace(int64_t bh, int32_t n, int32_t rank, int32_t ritz);
int spr_warm_metric_factor_ex(const float* metric, const float* prev_state, const float* prev_factor, int64_t bh,
                              int32_t n, int32_t rank, int32_t power_iters, int32_t ortho, int32_t ritz,
                              float rayleigh_ridge, float cqr_ridge, float* factor, float* state, uint8_t* recovered,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);
int spr_warm_metric_factor(const float* metric, const float* prev_state, const float* prev_factor, int64_t bh,
                           int32_t n, int32_t rank, int32_t power_iters, int32_t ortho, int32_t ritz,
                           float rayleigh_ridge, float cqr_ridge, float* factor, float* state, uint8_t* recovered,
                           hipStream_t stream);
/* operator_kmeans.py:534-555 project_tokens (+ normalize_rows_rms with row_rms = 1, eps 1e-6) and
 * n8_v6.py:152-178 the compiled K-centroid projection (tf32 = 1, div = the key scale):
 *   out fp32 [bh, m, r] = (x fp32 [bh, m, d] . factor fp32 [bh, d, r]) / div[h] (div nullable);
 *   d <= 128, r <= 64. */
int spr_project_rows(const float* x, const float* factor, const float* div, int64_t bh, int64_t m, int32_t d,
                     int32_t r, int32_t tf32, int32_t row_rms, float eps, float* out, hipStream_t stream);
/* The same with precision 0 fp32 / 1 TF32 / 2 bf16 operands (role_kv_matmul_precision
 * "highest" / "high" / "medium") and out[i][out_col + c] (rows of out_ld floats) = weight (p / div)
 * (the K and weighted V centroid projections of _role_kv_init_projection_fp32, n8_v6.py:118-126). */
int spr_project_rows_ex(const float* x, const float* factor, const float* div, int64_t bh, int64_t m, int32_t d,
                        int32_t r, int32_t precision, int32_t row_rms, float eps, float weight, float* out,
                        int32_t out_ld, int32_t out_col, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEPR_HIP_H */
