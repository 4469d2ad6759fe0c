"""SparsePR k-means / block-selection / block-sparse-attention entry points on HIP.

Drop-in for the parts of the reference's src/sparsepr/kmeans_utils.py on the
sparse-attention path: same names, arguments, return values and errors.
Every function runs the HIP kernels of libsparsepr_hip.so; none has a CPU
path (the reference's flash backends require CUDA tensors too).
"""

from __future__ import annotations

import torch

from .flash_kmeans.kmeans_impl import X_SQ_BF16, X_SQ_FP32, euclid_assign, lloyd
from .kernels import selection
from .kernels.permute import apply_inverse_permutation, argsort_labels, permute_tensor_by_labels


def _sizes(labels: torch.Tensor, n_clusters: int) -> torch.Tensor:
    return argsort_labels(labels.to(torch.int32), n_clusters)[1]


def _assign_only(x, init_centroids, n_clusters):
    """kmeans_utils.py:1212-1278: assign to fixed centroids (fp32 x_sq)."""
    if init_centroids is None:
        raise RuntimeError("Euclidean assign-only mode requires init_centroids.")
    if not x.is_cuda:
        raise RuntimeError(
            "Euclidean assign-only k-means requires a CUDA tensor "
            f"(device={x.device}). The chunked Python assign path was removed."
        )
    B, N, D = x.shape
    centroids = init_centroids.contiguous().view(B, n_clusters, D)
    labels = euclid_assign(x.contiguous(), centroids, None, x_sq_mode=X_SQ_FP32)
    return labels.long(), centroids, _sizes(labels, n_clusters).long(), 0


def _batch_kmeans_flash(x, n_clusters, max_iters, tol, init_centroids, verbose):
    """kmeans_utils.py:1372-1465: warm start -> inline fp32 x_sq; cold start ->
    flash_kmeans (x.dtype x_sq buffer).  Returns sizes as int64."""
    if max_iters == 0:
        return _assign_only(x, init_centroids, n_clusters)
    if not x.is_cuda:
        raise RuntimeError("Flash-KMeans backend requires a CUDA input tensor.")
    if x.ndim != 3:
        raise RuntimeError(f"Flash-KMeans expects [B, N, D] input, got shape {tuple(x.shape)}.")
    mode = X_SQ_FP32 if init_centroids is not None else X_SQ_BF16
    res = lloyd(x.contiguous(), n_clusters, max_iters, tol, init_centroids, x_sq_mode=mode, verbose=verbose)
    return res.labels, res.centroids, res.sizes.long(), int(res.iters)


def _batch_kmeans_n8_native(x, n_clusters, max_iters, init_centroids):
    """kmeans_utils.py:1468-1501: fixed-iteration exact-FP32 D64 Lloyd steps."""
    if not x.is_cuda or x.ndim != 3 or x.shape[2] != 64:
        raise RuntimeError("N8 CUDA role clustering requires CUDA X[BH,N,64].")
    if init_centroids is None:
        raise RuntimeError("N8 CUDA role clustering requires initialized centroids.")
    if max_iters <= 0:
        raise RuntimeError("N8 CUDA role clustering requires at least one iteration.")
    if n_clusters > 1024:
        raise RuntimeError("N8 CUDA role clustering supports at most 1024 clusters.")
    from .kernels.n8_extension import role_cluster_step_k64, role_cluster_step_q64

    x = x.float().contiguous()
    centroids = init_centroids.float().contiguous().view(x.shape[0], n_clusters, 64)
    step = role_cluster_step_q64 if n_clusters <= 512 else role_cluster_step_k64
    labels = sizes = None
    for _ in range(int(max_iters)):
        labels, centroids, sizes = step(x, centroids)
    return labels, centroids, sizes.long(), int(max_iters)


def _lloyd_result(x, n_clusters, max_iters=100, tol=1e-4, init_centroids=None, backend="cuvs"):
    """batch_kmeans_Euclid's loop returning the LloydResult, whose sorted_idx / offsets (the
    stable sort of the final labels) the N8 route reuses for its centroids and permutation."""
    from .flash_kmeans.kmeans_impl import LloydResult

    if backend == "n8_cuda_ext":
        labels, cent, _sizes, iters = _batch_kmeans_n8_native(x, n_clusters, max_iters, init_centroids)
        idx, sizes, offsets = argsort_labels(labels, n_clusters)
        return LloydResult(labels, cent, sizes, iters, idx, offsets)
    if backend not in ("flash", "cuvs"):
        raise RuntimeError(
            f"Unknown Euclidean k-means backend {backend!r}. "
            "Expected 'cuvs', 'flash', or 'n8_cuda_ext'."
        )
    if max_iters <= 0:
        raise RuntimeError("the route's k-means needs at least one iteration")
    if not x.is_cuda:
        raise RuntimeError("Flash-KMeans backend requires a CUDA input tensor.")
    mode = X_SQ_FP32 if (backend == "flash" and init_centroids is not None) else X_SQ_BF16
    return lloyd(x.contiguous(), n_clusters, max_iters, tol, init_centroids, x_sq_mode=mode)


def batch_kmeans_Euclid(x, n_clusters, max_iters=100, tol=1e-4, init_centroids=None, verbose=False,
                        backend="cuvs"):
    """Batched Euclidean k-means (kmeans_utils.py:1504-1580).

    Returns (cluster_ids, centroids [B,K,D] in x.dtype, cluster_sizes [B,K], n_iters).
    backend "cuvs" (the in-file path): int64 labels, int32 sizes, x.dtype x_sq;
    "flash": int32 labels, int64 sizes; "n8_cuda_ext": exact FP32 D=64 steps."""
    if max_iters < 0:
        raise RuntimeError(f"max_iters must be non-negative, got {max_iters}.")
    if backend == "flash":
        return _batch_kmeans_flash(x, n_clusters, max_iters, tol, init_centroids, verbose)
    if backend == "n8_cuda_ext":
        return _batch_kmeans_n8_native(x, n_clusters, max_iters, init_centroids)
    if backend != "cuvs":
        raise RuntimeError(
            f"Unknown Euclidean k-means backend {backend!r}. "
            "Expected 'cuvs', 'flash', or 'n8_cuda_ext'."
        )
    if max_iters == 0:
        return _assign_only(x, init_centroids, n_clusters)
    if not x.is_cuda:
        raise RuntimeError("k-means requires a GPU tensor (no CPU path).")
    res = lloyd(x.contiguous(), n_clusters, max_iters, tol, init_centroids, x_sq_mode=X_SQ_BF16,
                verbose=verbose)
    return res.labels.long(), res.centroids, res.sizes, int(res.iters)


def weighted_softmax(scores, weights):
    """w * exp(s - max) / max(sum, 1e-12) in fp32, returned in the input dtype
    (kmeans_utils.py:1698-1707).  Torch ops on the GPU; identify_dynamic_map
    does not call it (its fused kernel includes this step)."""
    input_dtype = scores.dtype
    scores = scores.float()
    weights = weights.float()
    max_score = torch.max(scores, dim=-1, keepdim=True)[0]
    weighted_exp = weights * torch.exp(scores - max_score)
    out = weighted_exp / torch.sum(weighted_exp, dim=-1, keepdim=True).clamp(min=1e-12)
    return out.to(input_dtype)


def identify_dynamic_map(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes, p, min_kc_ratio=0):
    """Top-p cluster-pair map (kmeans_utils.py:1710-1742): bool [B, H, Qc, Kc].

    One fused HIP kernel per (b, h, q-cluster): scores, size-weighted softmax,
    descending sort, cumulative mass, keep the prefix up to and including the
    first cluster that crosses p (and the first int(min_kc_ratio*Kc) ranks)."""
    del q_cluster_sizes  # the reference does not use it either
    B, H, qc_num, D = query_centroids.shape
    kc_num = key_centroids.shape[2]
    out = selection.topp_map(query_centroids.reshape(B * H, qc_num, D),
                             key_centroids.reshape(B * H, kc_num, D),
                             k_cluster_sizes.reshape(B * H, kc_num), p, min_kc_ratio)
    return out.view(B, H, qc_num, kc_num)


def density_calculation(dynamic_map, q_cluster_sizes, k_cluster_sizes):
    """Kept pairs / all pairs per (cfg, head) (kmeans_utils.py:285-303)."""
    return selection.density(dynamic_map, q_cluster_sizes, k_cluster_sizes)




def dynamic_block_sparse_fwd_flashinfer(q, k, v, block_mask_map, block_row_sz, block_col_sz, is_cpu=True,
                                        num_kv_heads=None, return_lse=False, plan_cache_key=None,
                                        plan_cache_token=None, selected_schedule=None):
    """Variable-block-sparse attention (kmeans_utils.py:2164-2350), HIP kernel.

    q [B, H_q, S, D], k/v [B, H_kv, S, D] bf16 in cluster order; block_mask_map
    [B, H_kv, Qc, Kc] bool; block_row_sz [B, H_kv, Qc], block_col_sz [B, H_kv, Kc].
    num_kv_heads enables GQA (query head h uses kv head h // (H_q / H_kv)).
    return_lse adds the natural-log LSE [B, H_q, S] (fp32).  plan_cache_key /
    plan_cache_token reuse the kept-segment plan while the token is unchanged.
    selected_schedule = (ids [B, H_kv, Qc, Kc], counts [B, H_kv, Qc]), the selector's
    ascending kept-cluster schedule (svg_ear_select_budget_schedule), builds the plan
    from the schedule instead of scanning the map (the same plan when both agree)."""
    from .kernels.attention import block_sparse_attention, cached_plan

    B, H_q, S, D = q.shape
    if num_kv_heads is not None:
        H_kv = num_kv_heads
        assert k.shape[1] == H_kv and v.shape[1] == H_kv, (
            f"GQA-native: K/V must have {H_kv} heads, got K={k.shape[1]}, V={v.shape[1]}"
        )
        assert H_q % H_kv == 0, f"Q heads ({H_q}) must be divisible by KV heads ({H_kv})"
    else:
        H_kv = H_q
        assert k.shape[1] == H_q and v.shape[1] == H_q
    qc_num = block_row_sz.shape[-1]
    kc_num = block_col_sz.shape[-1]
    assert block_mask_map.shape == (B, H_kv, qc_num, kc_num)
    assert (
        all(t.device == torch.device("cpu") for t in [block_mask_map, block_row_sz, block_col_sz]) if is_cpu else True
    )
    dev = q.device
    bmap = block_mask_map.reshape(B * H_kv, qc_num, kc_num).to(dev)
    rows = block_row_sz.reshape(B * H_kv, qc_num).to(dev)
    cols = block_col_sz.reshape(B * H_kv, kc_num).to(dev)
    plan = None
    if selected_schedule is not None:
        if plan_cache_key is not None:
            raise ValueError("selected_schedule and plan_cache_key are exclusive.")
        from .kernels.attention import plan_block_sparse_from_schedule

        ids, counts = selected_schedule
        plan = plan_block_sparse_from_schedule(ids.reshape(B * H_kv, qc_num, kc_num),
                                               counts.reshape(B * H_kv, qc_num), rows, cols, S)
    elif plan_cache_key is not None:
        if plan_cache_token is None:
            raise ValueError("plan_cache_token is required when plan_cache_key is set.")
        plan = cached_plan(plan_cache_key, plan_cache_token, bmap, rows, cols, S)
    res = block_sparse_attention(q.reshape(B * H_q, S, D), k.reshape(B * H_kv, S, D), v.reshape(B * H_kv, S, D),
                                 bmap, rows, cols, return_lse=return_lse, plan=plan)
    if return_lse:
        o, lse = res
        return o.reshape(B, H_q, S, D), lse.reshape(B, H_q, S)
    return res.reshape(B, H_q, S, D)


def dynamic_block_sparse_fwd_triton(q, k, v, dynamic_map, qc_size, kc_size):
    """Same computation as the reference's Triton variant (kmeans_utils.py:1847-2161)."""
    return dynamic_block_sparse_fwd_flashinfer(q, k, v, dynamic_map, qc_size, kc_size, is_cpu=False)
