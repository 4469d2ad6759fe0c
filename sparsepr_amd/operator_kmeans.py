"""Operator-induced role metrics, their factors and original-space centroids for the N8
router (drop-in for src/sparsepr/models/cosmos3/operator_kmeans.py on the route's path).

Every computation runs on the HIP kernels of libsparsepr_hip.so (csrc/spr_metric.hip,
csrc/spr_rrr.hip, csrc/spr_kmeans.hip); there is no CPU path.  Names, arguments and error
messages follow the reference.  Not provided: the legacy_fp32 / tensorcore_fp32 backend
switch (the kernels accumulate bf16 / fp32 products in fp32, the reference's contract for
both), the each_qr / final_qr Householder orthogonalisations and the "full" Ritz mode of
warm_subspace_metric_factor (they raise NotImplementedError), lift_projected_centroids and
metric_relative_drift (diagnostics, not on the route).
"""

from __future__ import annotations

import torch

from .kernels import role_metric as _rm

_POSITIONS: dict = {}


def deterministic_token_positions(tokens: int, sample_tokens: int, device) -> torch.Tensor | None:
    """The sample of deterministic_token_sample (operator_kmeans.py:52-59): round(linspace(0,
    N - 1, sample_tokens)) made unique, computed by torch on the tensors' device (the
    reference's own op sequence) and cached per (N, samples, device).  None = all rows."""
    if sample_tokens <= 0 or sample_tokens >= tokens:
        return None
    key = (int(tokens), int(sample_tokens), str(device))
    pos = _POSITIONS.get(key)
    if pos is None:
        lin = torch.linspace(0, tokens - 1, steps=sample_tokens, device=device)
        pos = lin.round().long().unique(sorted=True).to(torch.int32).contiguous()
        _POSITIONS[key] = pos
    return pos


def deterministic_token_sample(x: torch.Tensor, sample_tokens: int) -> torch.Tensor:
    if x.ndim != 3:
        raise RuntimeError(f"Expected [batch_heads, tokens, dim], got {tuple(x.shape)}.")
    pos = deterministic_token_positions(int(x.shape[1]), sample_tokens, x.device)
    if pos is None:
        return x
    from .flash_kmeans.kmeans_impl import gather_rows

    return gather_rows(x, pos.unsqueeze(0).expand(x.shape[0], -1))


def covariance(x: torch.Tensor, *, center: bool) -> torch.Tensor:
    """fp32 (x - mean)^T (x - mean) / N (or x^T x / N), operator_kmeans.py:62-92."""
    if x.ndim != 3:
        raise RuntimeError(f"Expected [batch_heads, tokens, dim], got {tuple(x.shape)}.")
    return _rm.role_metric(x, center=center)


def key_metric_from_queries(queries: torch.Tensor, sample_tokens: int) -> torch.Tensor:
    """Uncentred second moment of the deterministic sample of the queries (:491-493)."""
    if queries.ndim != 3:
        raise RuntimeError(f"Expected [batch_heads, tokens, dim], got {tuple(queries.shape)}.")
    pos = deterministic_token_positions(int(queries.shape[1]), sample_tokens, queries.device)
    return _rm.role_metric(queries, rows=pos, center=False)


def value_metric_from_values(values: torch.Tensor, sample_tokens: int) -> torch.Tensor:
    """Centred covariance of the deterministic sample of the values (:496-498)."""
    if values.ndim != 3:
        raise RuntimeError(f"Expected [batch_heads, tokens, dim], got {tuple(values.shape)}.")
    pos = deterministic_token_positions(int(values.shape[1]), sample_tokens, values.device)
    return _rm.role_metric(values, rows=pos, center=True)


def query_metric_from_key_centroids(centroids: torch.Tensor, sizes: torch.Tensor) -> torch.Tensor:
    """Centred full-logit metric of the non-empty key centroids, / D (:517-531)."""
    if centroids.ndim != 3 or sizes.shape != centroids.shape[:2]:
        raise RuntimeError(
            f"Centroid metric shape mismatch: centroids={tuple(centroids.shape)}, sizes={tuple(sizes.shape)}."
        )
    return _rm.role_metric(centroids.float(), sizes=sizes, center=True, post_scale=1.0 / float(centroids.shape[-1]))


def metric_factor(metric: torch.Tensor, rank: int) -> torch.Tensor:
    """Top-rank eigenvectors of the symmetrised metric scaled by sqrt(lambda / mean lambda),
    fp32 (:95-151).  Non-finite metrics raise, as the reference does before its eigh."""
    if metric.ndim != 3 or metric.shape[1] != metric.shape[2]:
        raise RuntimeError(f"Expected batched square metrics, got {tuple(metric.shape)}.")
    if rank <= 0 or rank > metric.shape[-1]:
        raise RuntimeError(f"rank must be in [1, {metric.shape[-1]}], got {rank}.")
    if rank > 64 or metric.shape[-1] > 128:
        raise NotImplementedError("metric_factor on the MI355X kernels supports D <= 128 and rank <= 64.")
    if not bool(torch.isfinite(metric).all()):
        raise RuntimeError("Role metric contains non-finite values before factorization.")
    return _rm.metric_factor(metric, int(rank))


def warm_subspace_metric_factor(metric, previous_factor, rank, *, power_iters=1, orthogonalization="each_qr",
                                ritz_mode="full", rayleigh_ridge=1e-6, cholesky_qr_ridge=1e-4, return_basis=False,
                                return_recovery_mask=False):
    """Subspace-iteration update of a previous top-r factor (:219-477), one fused kernel per
    call (three with the full finish: the subspace kernel, the reduced eigensolver, the
    factor).  Returns factor, or (factor, basis[, recovery_mask]) as the reference."""
    if metric.ndim != 3 or metric.shape[1] != metric.shape[2]:
        raise RuntimeError(f"Expected batched square metrics, got {tuple(metric.shape)}.")
    if rank <= 0 or rank > metric.shape[-1]:
        raise RuntimeError(f"rank must be in [1, {metric.shape[-1]}], got {rank}.")
    expected = (metric.shape[0], metric.shape[1], rank)
    if tuple(previous_factor.shape) != expected:
        raise RuntimeError(
            f"Previous factor shape mismatch: got {tuple(previous_factor.shape)}, expected {expected}."
        )
    if power_iters < 1:
        raise RuntimeError(f"power_iters must be positive, got {power_iters}.")
    if rayleigh_ridge <= 0.0:
        raise RuntimeError(f"rayleigh_ridge must be positive, got {rayleigh_ridge}.")
    if cholesky_qr_ridge <= 0.0:
        raise RuntimeError(f"cholesky_qr_ridge must be positive, got {cholesky_qr_ridge}.")
    if orthogonalization not in {"each_qr", "final_qr", "cholesky_qr", "each_cholesky_qr", "each_cholesky_qr2"}:
        raise RuntimeError(f"Unknown subspace orthogonalization {orthogonalization!r}.")
    if ritz_mode not in {"full", "rayleigh_cholesky", "diagonal", "previous_scale"}:
        raise RuntimeError(f"Unknown Rayleigh--Ritz mode {ritz_mode!r}.")
    if rank > 64 or metric.shape[-1] > 128:
        raise NotImplementedError("warm_subspace_metric_factor on the MI355X kernels supports D <= 128, rank <= 64.")
    factor, basis, rec = _rm.warm_metric_factor(
        metric, previous_factor, int(rank), power_iters=int(power_iters), orthogonalization=orthogonalization,
        ritz_mode=ritz_mode, rayleigh_ridge=rayleigh_ridge, cholesky_qr_ridge=cholesky_qr_ridge)
    if return_basis and return_recovery_mask:
        return factor, basis, rec
    if return_basis:
        return factor, basis
    if return_recovery_mask:
        raise ValueError("return_recovery_mask requires return_basis=True.")
    return factor


def key_factor_from_queries(queries: torch.Tensor, rank: int, sample_tokens: int) -> torch.Tensor:
    return metric_factor(key_metric_from_queries(queries, sample_tokens), rank)


def value_factor_from_values(values: torch.Tensor, rank: int, sample_tokens: int) -> torch.Tensor:
    return metric_factor(value_metric_from_values(values, sample_tokens), rank)


def query_factor_from_key_centroids(centroids: torch.Tensor, sizes: torch.Tensor, rank: int) -> torch.Tensor:
    return metric_factor(query_metric_from_key_centroids(centroids, sizes), rank)


def project_tokens(x: torch.Tensor, factor: torch.Tensor) -> torch.Tensor:
    """fp32 x . factor (:534-538)."""
    if x.ndim != 3 or factor.ndim != 3 or x.shape[0] != factor.shape[0] or x.shape[2] != factor.shape[1]:
        raise RuntimeError(f"Projection shape mismatch: x={tuple(x.shape)}, factor={tuple(factor.shape)}.")
    return _rm.project_rows(x, factor)


def gqa_metric_sources(q: torch.Tensor, k: torch.Tensor, *, q_cluster_heads: int, k_cluster_heads: int,
                       gqa_group_size: int):
    """K samples for the Q metric and Q samples for the K metric (:558-606)."""
    if q.ndim != 4 or k.ndim != 4 or q.shape != k.shape:
        raise RuntimeError(f"Expected matching [B,H,N,D] Q/K tensors, got Q={tuple(q.shape)}, K={tuple(k.shape)}.")
    batch, heads, tokens, dim = q.shape
    if gqa_group_size <= 0:
        raise RuntimeError(f"gqa_group_size must be positive, got {gqa_group_size}.")
    if q_cluster_heads == heads:
        q_metric_keys = k.contiguous().view(batch * heads, tokens, dim)
    elif q_cluster_heads * gqa_group_size == heads:
        q_metric_keys = k[:, ::gqa_group_size].contiguous().view(batch * q_cluster_heads, tokens, dim)
    else:
        raise RuntimeError(
            f"Cannot construct Q metrics for heads={heads}, q_cluster_heads={q_cluster_heads}, G={gqa_group_size}."
        )
    if k_cluster_heads == heads:
        k_metric_queries = q.contiguous().view(batch * heads, tokens, dim)
    elif k_cluster_heads * gqa_group_size == heads:
        k_metric_queries = q.contiguous().view(batch * k_cluster_heads, gqa_group_size * tokens, dim)
    else:
        raise RuntimeError(
            f"Cannot construct K metrics for heads={heads}, k_cluster_heads={k_cluster_heads}, G={gqa_group_size}."
        )
    return q_metric_keys, k_metric_queries


def _sorted_labels(labels: torch.Tensor, clusters: int):
    from .kernels.permute import argsort_labels

    idx, _sizes, offsets = argsort_labels(labels.to(torch.int32).contiguous(), clusters)
    return idx, offsets


def _check_centroid_inputs(x, labels, cluster_sizes):
    if x.ndim != 3 or labels.shape != x.shape[:2]:
        raise RuntimeError(f"Centroid shape mismatch: x={tuple(x.shape)}, labels={tuple(labels.shape)}.")
    if cluster_sizes.shape[0] != x.shape[0]:
        raise RuntimeError(
            f"Cluster-size shape mismatch: sizes={tuple(cluster_sizes.shape)}, batch_heads={x.shape[0]}."
        )


def original_centroids(x: torch.Tensor, labels: torch.Tensor, cluster_sizes: torch.Tensor, *,
                       empty_fallback: torch.Tensor | None = None, sorted_labels=None) -> torch.Tensor:
    """fp32 means of x under labels; empty clusters take empty_fallback (zeros when None)
    (:609-642).  The sums are fp64, so the result does not depend on the summation order.
    `sorted_labels` = (sorted_idx, offsets) of the labels when the caller has them."""
    _check_centroid_inputs(x, labels, cluster_sizes)
    clusters = int(cluster_sizes.shape[1])
    idx, offsets = sorted_labels if sorted_labels is not None else _sorted_labels(labels, clusters)
    return _rm.original_centroids(x, None, idx, offsets, clusters, x_fallback=empty_fallback)


def joint_original_centroids(x: torch.Tensor, y: torch.Tensor, labels: torch.Tensor, cluster_sizes: torch.Tensor, *,
                             x_empty_fallback: torch.Tensor | None = None,
                             y_empty_fallback: torch.Tensor | None = None, sorted_labels=None):
    """Means of x and y under one traversal of the sorted labels (:645-679)."""
    _check_centroid_inputs(x, labels, cluster_sizes)
    clusters = int(cluster_sizes.shape[1])
    idx, offsets = sorted_labels if sorted_labels is not None else _sorted_labels(labels, clusters)
    return _rm.original_centroids(x, y, idx, offsets, clusters, x_fallback=x_empty_fallback,
                                  y_fallback=y_empty_fallback)


def role_metric_backend() -> str:
    """The kernels accumulate products of the bf16 / fp32 inputs in fp32 (both reference
    backends' contract); the name reports the reference default."""
    return "legacy_fp32"


def original_centroid_backend() -> str:
    return "triton_atomic_fp32"


__all__ = [
    "deterministic_token_positions", "deterministic_token_sample", "covariance", "key_metric_from_queries",
    "value_metric_from_values", "query_metric_from_key_centroids", "metric_factor", "warm_subspace_metric_factor",
    "key_factor_from_queries", "value_factor_from_values", "query_factor_from_key_centroids", "project_tokens",
    "gqa_metric_sources", "original_centroids", "joint_original_centroids",
]
