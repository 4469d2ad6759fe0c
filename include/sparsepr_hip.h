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
 *   labels int32 [batch, n]; d in {64, 128}. */
int spr_kmeans_assign_bf16(const void* x, const void* centroids, const float* c_sq, const float* x_sq,
                           int32_t x_sq_mode, int64_t batch, int64_t n, int32_t k, int32_t d, int32_t* labels,
                           hipStream_t stream);
/* centroid_update_triton.py:316-386 triton_centroid_update_sorted_euclid,
 * centroid_reduction.py:138-196 original_centroids_triton, n8_ops.cu:255-269 finalize.
 *   Means of the rows of each cluster (sorted_idx/offsets from spr_argsort_labels), fp64
 *   accumulation, empty clusters keep `old`.  dtype 0 (bf16, d in {64,128}) or 2 (fp32,
 *   d in {16,32,48,64,128}).  Nullable outputs: mean32 fp32 [batch,k,d], out dtype [batch,k,d],
 *   shift_max fp32 scalar (pre-zeroed; max_k ||out-old||), sums_accum fp32 += sums,
 *   counts_accum int32 += counts. */
int spr_centroid_mean(const void* x, int32_t dtype, const int32_t* sorted_idx, const int32_t* offsets,
                      const void* old, int64_t batch, int64_t n, int32_t k, int32_t d, float* mean32, void* out,
                      float* shift_max, float* sums_accum, int32_t* counts_accum, hipStream_t stream);
/* n8_ops.cu:198-253 role_cluster_assign_accumulate_q64_kernel (assignment part):
 *   exact FP32 distance (sequential fmaf), lowest index on ties; d in {16,32,48,64}.
 *   best_dist nullable. */
int spr_role_assign_fp32(const float* features, const float* centroids, int64_t batch, int64_t n, int32_t k,
                         int32_t d, int32_t* labels, float* best_dist, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEPR_HIP_H */
