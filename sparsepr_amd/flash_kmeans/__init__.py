"""Batched flash k-means on HIP (drop-in for the reference's src/flash_kmeans).

Public names follow the reference package (flash_kmeans/__init__.py:37-46);
the Triton kernels are replaced by the HIP kernels of csrc/spr_kmeans.hip and
csrc/spr_sort.hip.  There is no torch fallback: without the built library or a
GPU these functions raise.
"""

from __future__ import annotations

import torch

from .interface import FlashKMeans
from .kmeans_impl import (
    X_SQ_BF16,
    X_SQ_FP32,
    centroid_sq,
    centroid_update_sorted,
    euclid_assign,
    lloyd,
)


def batch_kmeans_Euclid(x, n_clusters, max_iters=100, tol=0.0, init_centroids=None, verbose=False, *,
                        use_heuristic=True):
    """Batched Lloyd k-means (reference kmeans_triton_impl.py:55-115).

    x [B, N, D] bf16 (or fp32); returns (cluster_ids int32 [B, N], centroids [B, K, D]
    in x.dtype, iterations run).  x_sq follows the reference's x.dtype buffer."""
    del use_heuristic
    res = lloyd(x, n_clusters, max_iters, tol, init_centroids, x_sq_mode=X_SQ_BF16, verbose=verbose)
    return res.labels, res.centroids, res.iters


def euclid_assign_triton(x, centroids, x_sq, out=None, c_sq=None, *, BLOCK_N=128, BLOCK_K=128,
                         num_warps=None, num_stages=None, config=None, use_heuristic=True):
    """Nearest-centroid ids int32 [B, N] (reference assign_euclid_triton.py:1238-1412).

    x_sq [B, N] is used as given (any float dtype); c_sq defaults to fp32 ||c||^2."""
    del BLOCK_N, BLOCK_K, num_warps, num_stages, config, use_heuristic
    return euclid_assign(x, centroids, x_sq, c_sq=c_sq, out=out)


def triton_centroid_update_sorted_euclid(x, cluster_ids, old_centroids, *, BLOCK_N=256, centroid_sums=None,
                                         centroid_cnts=None, calculate_new=True):
    """Cluster means; empty clusters keep the old centroid (centroid_update_triton.py:316-386).

    When given, centroid_sums (fp32 [B,K,D]) and centroid_cnts (int32 [B,K]) are
    accumulated into, as the reference's atomics do."""
    del BLOCK_N
    res = centroid_update_sorted(x, cluster_ids, old_centroids, sums_accum=centroid_sums,
                                 counts_accum=centroid_cnts)
    return res.centroids if calculate_new else None


def triton_centroid_update_euclid(x, cluster_ids, old_centroids):
    """Same result as the sorted variant (the reference's per-token atomic kernel)."""
    return triton_centroid_update_sorted_euclid(x, cluster_ids, old_centroids)


__all__ = [
    "batch_kmeans_Euclid",
    "euclid_assign_triton",
    "triton_centroid_update_euclid",
    "triton_centroid_update_sorted_euclid",
    "FlashKMeans",
    "centroid_sq",
]

__version__ = "0.3.1+mi355x"
