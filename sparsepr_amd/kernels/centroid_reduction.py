"""Original-space cluster means (drop-in for src/sparsepr/kernels/triton/centroid_reduction.py:
original_centroids_triton / joint_original_centroids_triton, :138-196) on the HIP
original_mean_kernel: fp64 sums read through the stable label sort, one traversal for
both tensors of the joint form, fp32 means, empty clusters from the fallback (zeros
without one)."""

from __future__ import annotations

import torch

from .. import _lib
from . import role_metric as _rm


def _validate(x, labels, sizes, fallback):
    if x.ndim != 3 or labels.shape != x.shape[:2]:
        raise RuntimeError(f"Centroid shape mismatch: x={tuple(x.shape)}, labels={tuple(labels.shape)}.")
    if sizes.ndim != 2 or sizes.shape[0] != x.shape[0]:
        raise RuntimeError(f"Cluster-size shape mismatch: sizes={tuple(sizes.shape)}, batch_heads={x.shape[0]}.")
    if fallback is not None and tuple(fallback.shape) != (x.shape[0], sizes.shape[1], x.shape[2]):
        raise RuntimeError(
            f"Empty-centroid fallback mismatch: fallback={tuple(fallback.shape)}, "
            f"means={(x.shape[0], sizes.shape[1], x.shape[2])}.")
    _lib.require_gpu(x, labels, sizes, fallback, what="original centroids")
    return int(sizes.shape[1])


def _sorted(labels, clusters):
    from .permute import argsort_labels

    idx, _s, offsets = argsort_labels(labels.to(torch.int32).contiguous(), clusters)
    return idx, offsets


def original_centroids_triton(x: torch.Tensor, labels: torch.Tensor, sizes: torch.Tensor, *,
                              empty_fallback: torch.Tensor | None = None) -> torch.Tensor:
    clusters = _validate(x, labels, sizes, empty_fallback)
    idx, offsets = _sorted(labels, clusters)
    return _rm.original_centroids(x, None, idx, offsets, clusters, x_fallback=empty_fallback)


def joint_original_centroids_triton(x: torch.Tensor, y: torch.Tensor, labels: torch.Tensor, sizes: torch.Tensor, *,
                                    x_empty_fallback: torch.Tensor | None = None,
                                    y_empty_fallback: torch.Tensor | None = None):
    clusters = _validate(x, labels, sizes, x_empty_fallback)
    _validate(y, labels, sizes, y_empty_fallback)
    if y.shape != x.shape:
        raise RuntimeError(f"Joint centroid inputs differ: X={tuple(x.shape)}, Y={tuple(y.shape)}.")
    idx, offsets = _sorted(labels, clusters)
    return _rm.original_centroids(x, y, idx, offsets, clusters, x_fallback=x_empty_fallback,
                                  y_fallback=y_empty_fallback)
