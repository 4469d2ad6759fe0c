"""Native N8 kernels (drop-in for the reference's src/sparsepr/kernels/n8_extension.py).

The reference loads a pybind module `n8_kernels` built from n8_ops.cu.  Here the
same entry points are served by libsparsepr_hip.so through its C ABI.
`load_n8_kernels()` returns a module-like object exposing the reference's export
names (n8_ops.cu:642-664) so `hasattr` capability probes keep working; the
model-specific QKV norm/RoPE fusions are not part of this library.
"""

from __future__ import annotations

import types

import torch

from .. import _lib

_MODULE: types.SimpleNamespace | None = None
_LOAD_ERROR: Exception | None = None


def _check_role_inputs(features, centroids, max_clusters):
    _lib.require_gpu(features, centroids, what="role clustering")
    if features.dtype != torch.float32 or centroids.dtype != torch.float32:
        raise RuntimeError("Role clustering requires FP32 features and centroids")
    if not (features.is_contiguous() and centroids.is_contiguous()):
        raise RuntimeError("Role clustering inputs must be contiguous")
    if (features.dim() != 3 or centroids.dim() != 3 or features.shape[0] != centroids.shape[0]
            or features.shape[2] != 64 or centroids.shape[2] != 64):
        raise RuntimeError("Role clustering expects features [BH,N,64], centroids [BH,C,64]")
    clusters = centroids.shape[1]
    if not 0 < clusters <= max_clusters:
        raise RuntimeError("Unsupported role cluster count")


def _role_step(features: torch.Tensor, centroids: torch.Tensor, max_clusters: int):
    """One exact FP32 Lloyd step: assign, sizes, means (n8_ops.cu:499-529)."""
    _check_role_inputs(features, centroids, max_clusters)
    from ..flash_kmeans.kmeans_impl import centroid_update_sorted
    from .permute import argsort_labels

    bh, n, d = features.shape
    c = centroids.shape[1]
    labels = torch.empty((bh, n), dtype=torch.int32, device=features.device)
    # exact FP32 distances, sequential fmaf over the dims (n8_ops.cu:189-253), not TF32
    _lib.call("spr_role_assign_fp32", _lib.ptr(features), _lib.ptr(centroids), bh, n, c, d, _lib.ptr(labels), None,
              _lib.stream(features.device))
    idx, sizes, offsets = argsort_labels(labels, c)
    res = centroid_update_sorted(features, labels, centroids, sorted_idx=idx, sizes=sizes, offsets=offsets)
    return [labels, res.centroids, sizes]


def role_cluster_step_q64(features: torch.Tensor, centroids: torch.Tensor):
    """[labels int32, centroids fp32, sizes int32] for at most 512 clusters."""
    return tuple(_role_step(features, centroids, 512))


def role_cluster_step_k64(features: torch.Tensor, centroids: torch.Tensor):
    """[labels int32, centroids fp32, sizes int32] for at most 1024 clusters."""
    return tuple(_role_step(features, centroids, 1024))


def svg_ear_select_budget(scores: torch.Tensor, cluster_sizes: torch.Tensor,
                          budgets: torch.Tensor) -> torch.Tensor:
    """Exact descending selector budget and bool-mask scatter (n8_ops.cu:541-571)."""
    from .selection import MODE_N8_NATIVE, select_budget

    _lib.require_gpu(scores, cluster_sizes, budgets, what="Selector inputs")
    return select_budget(scores.contiguous(), cluster_sizes, budgets, MODE_N8_NATIVE)


def svg_ear_select_budget_schedule(scores: torch.Tensor, cluster_sizes: torch.Tensor,
                                   budgets: torch.Tensor):
    """Selector plus ascending fixed-stride selected-cluster ids and counts (n8_ops.cu:573-615)."""
    from .selection import MODE_N8_NATIVE, select_budget

    _lib.require_gpu(scores, cluster_sizes, budgets, what="Selector inputs")
    return tuple(select_budget(scores.contiguous(), cluster_sizes, budgets, MODE_N8_NATIVE,
                               with_schedule=True))


def compact_selected_clusters(selected_mask: torch.Tensor):
    """Ascending fixed-stride cluster ids and a count for every row (n8_ops.cu:617-638)."""
    from .selection import compact

    return tuple(compact(selected_mask))


def _exports() -> dict:
    return {
        "role_cluster_step_q64": lambda f, c: _role_step(f, c, 512),
        "role_cluster_step_k64": lambda f, c: _role_step(f, c, 1024),
        "svg_ear_select_budget": svg_ear_select_budget,
        "svg_ear_select_budget_schedule": lambda s, z, b: list(svg_ear_select_budget_schedule(s, z, b)),
        "compact_selected_clusters": lambda m: list(compact_selected_clusters(m)),
    }


def load_n8_kernels(*, required: bool = False):
    """Module-like view of the native kernels, or None when the library cannot
    be loaded and `required` is False (reference n8_extension.py:24-42)."""
    global _MODULE, _LOAD_ERROR
    if _MODULE is not None:
        return _MODULE
    if _LOAD_ERROR is not None and not required:
        return None
    try:
        _lib.load()
    except Exception as exc:  # missing or stale library
        _LOAD_ERROR = exc
        if required:
            raise RuntimeError(f"Could not load {_lib.LIB_PATH.name}: {exc}") from exc
        return None
    _MODULE = types.SimpleNamespace(**_exports())
    return _MODULE


def n8_cuda_extension_available() -> bool:
    return load_n8_kernels(required=False) is not None
