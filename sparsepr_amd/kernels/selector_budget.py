"""Exact full-width selector budget (drop-in for the reference's
src/sparsepr/kernels/triton/selector_budget.py:131-171) on csrc/spr_select.hip."""

from __future__ import annotations

import torch

from .selection import MODE_TRITON, select_budget


def exact_budget_dynamic_map_triton(scores: torch.Tensor, cluster_sizes: torch.Tensor,
                                    budgets: torch.Tensor) -> torch.Tensor:
    """Argsort (descending, ties by index) + prefix-budget keep + first crossing;
    bool [BH, Q+1, K+1] with the header row/column."""
    if not scores.is_cuda:
        raise RuntimeError("The exact selector-budget kernel requires CUDA tensors.")
    if scores.ndim != 3 or cluster_sizes.ndim != 2 or budgets.ndim != 2:
        raise RuntimeError("Expected scores [BH,Q,K], sizes [BH,K], budgets [BH,Q].")
    bh, q_clusters, k_clusters = scores.shape
    if tuple(cluster_sizes.shape) != (bh, k_clusters):
        raise RuntimeError("Key-cluster sizes do not match selector scores.")
    if tuple(budgets.shape) != (bh, q_clusters):
        raise RuntimeError("Per-query budgets do not match selector scores.")
    if k_clusters > 4096:
        raise RuntimeError(f"Exact selector supports at most 4096 key clusters, got {k_clusters}.")
    return select_budget(scores.float(), cluster_sizes, budgets, MODE_TRITON)
