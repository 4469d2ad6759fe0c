"""Block selection on the HIP kernels of csrc/spr_select.hip (shared by
kmeans_utils, selector_budget and n8_extension)."""

from __future__ import annotations

import math

import torch

from .. import _lib

MODE_N8_NATIVE = 0   # n8_ops.cu:271-322 semantics
MODE_TRITON = 1      # selector_budget.py:10-54 semantics


def topp_map(qc: torch.Tensor, kc: torch.Tensor, k_sizes: torch.Tensor, p: float,
             min_kc_ratio: float = 0.0) -> torch.Tensor:
    """qc [R, Qc, D], kc [R, Kc, D], k_sizes [R, Kc] -> bool [R, Qc, Kc]."""
    dev = _lib.require_gpu(qc, kc, k_sizes, what="identify_dynamic_map")
    r, qn, d = qc.shape
    kn = kc.shape[1]
    if kc.shape != (r, kn, d) or tuple(k_sizes.shape) != (r, kn):
        raise RuntimeError(f"top-p map shape mismatch: qc={tuple(qc.shape)} kc={tuple(kc.shape)} "
                           f"sizes={tuple(k_sizes.shape)}")
    score_bf16 = 1 if (qc.dtype == torch.bfloat16 and kc.dtype == torch.bfloat16) else 0
    q32 = qc.float().contiguous()
    k32 = kc.float().contiguous()
    ks = k_sizes.to(torch.int32).contiguous()
    preserve = int(min_kc_ratio * kn) if min_kc_ratio > 0 else 0
    out = torch.empty((r, qn, kn), dtype=torch.bool, device=dev)
    _lib.call("spr_topp_map", _lib.ptr(q32), _lib.ptr(k32), _lib.ptr(ks), r, qn, kn, d,
              float(math.sqrt(d)), float(p), preserve, score_bf16, _lib.ptr(out), None, _lib.stream(dev))
    return out


def top_p_key_budgets(q_centroids: torch.Tensor, k_centroids: torch.Tensor, k_cluster_sizes: torch.Tensor,
                      top_p: float) -> torch.Tensor:
    """SVG2 key-token budget of each query cluster (n8_v6.py:181-230): the summed sizes
    of the key clusters that the fp32 top-p rule keeps (rank 0 always, then every rank
    whose preceding cumulative mass is <= top_p).  [BH, Qc, D] x [BH, Kc, D] -> int64
    [BH, Qc].  The fp32 chain is the top-p map's (the same kernel, map not written)."""
    if q_centroids.ndim != 3 or k_centroids.ndim != 3:
        raise ValueError("TopP budget centroids must be [BH,C,D].")
    if q_centroids.shape[0] != k_centroids.shape[0]:
        raise ValueError("TopP Q/K centroids must have the same head count.")
    if q_centroids.shape[2] != k_centroids.shape[2]:
        raise ValueError("TopP Q/K centroids must have the same head dimension.")
    if tuple(k_cluster_sizes.shape) != tuple(k_centroids.shape[:2]):
        raise ValueError(
            "TopP K-cluster sizes must match K centroids, got "
            f"sizes={tuple(k_cluster_sizes.shape)} centroids={tuple(k_centroids.shape)}.")
    if not 0.0 < float(top_p) <= 1.0:
        raise ValueError(f"svg_ear_top_p must be in (0,1], got {top_p}.")
    dev = _lib.require_gpu(q_centroids, k_centroids, k_cluster_sizes, what="top-p key budgets")
    r, qn, d = q_centroids.shape
    kn = k_centroids.shape[1]
    q32 = q_centroids.float().contiguous()
    k32 = k_centroids.float().contiguous()
    ks = k_cluster_sizes.to(torch.int32).contiguous()
    budgets = torch.empty((r, qn), dtype=torch.int32, device=dev)
    _lib.call("spr_topp_map", _lib.ptr(q32), _lib.ptr(k32), _lib.ptr(ks), r, qn, kn, d, float(math.sqrt(d)),
              float(top_p), 0, 0, None, _lib.ptr(budgets), _lib.stream(dev))
    return budgets.long()


def select_budget(scores: torch.Tensor, sizes: torch.Tensor, budgets: torch.Tensor, mode: int,
                  with_schedule: bool = False):
    """scores fp32 [BH, Q, K], sizes [BH, K], budgets [BH, Q] -> bool [BH, Q+1, K+1]
    (and ascending kept ids int32 [BH, Q, K] + counts int32 [BH, Q] with_schedule)."""
    dev = _lib.require_gpu(scores, sizes, budgets, what="budget selector")
    if scores.dtype != torch.float32 or scores.dim() != 3:
        raise RuntimeError("Selector scores must be contiguous FP32 [BH,Q,K]")
    bh, qn, kn = scores.shape
    if sizes.dim() != 2 or tuple(sizes.shape) != (bh, kn):
        raise RuntimeError("Selector cluster-size shape mismatch")
    if budgets.dim() != 2 or tuple(budgets.shape) != (bh, qn):
        raise RuntimeError("Selector budget shape mismatch")
    sc = scores.contiguous()
    sz = sizes.to(device=dev, dtype=torch.int32).contiguous()
    bu = budgets.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty((bh, qn + 1, kn + 1), dtype=torch.bool, device=dev)
    ids = counts = None
    if with_schedule:
        ids = torch.empty((bh, qn, kn), dtype=torch.int32, device=dev)
        counts = torch.empty((bh, qn), dtype=torch.int32, device=dev)
    _lib.call("spr_select_budget", _lib.ptr(sc), _lib.ptr(sz), _lib.ptr(bu), bh, qn, kn, int(mode),
              _lib.ptr(out), _lib.ptr(ids), _lib.ptr(counts), _lib.stream(dev))
    if with_schedule:
        return out, ids, counts
    return out


def compact(mask: torch.Tensor):
    """bool [..., K] -> (ascending kept ids int32 [..., K], counts int32 [...])."""
    dev = _lib.require_gpu(mask, what="compact_selected_clusters")
    if mask.dtype != torch.bool:
        raise RuntimeError("Selected-cluster compaction requires a CUDA bool tensor")
    if mask.dim() < 2:
        raise RuntimeError("Selected-cluster compaction expects [...,K]")
    m = mask.contiguous()
    kn = m.shape[-1]
    if not 0 < kn <= 4096:
        raise RuntimeError("Selected-cluster compaction supports 1..4096 K clusters")
    rows = m.numel() // kn
    ids = torch.empty(m.shape, dtype=torch.int32, device=dev)
    counts = torch.empty(m.shape[:-1], dtype=torch.int32, device=dev)
    _lib.call("spr_compact_selected", _lib.ptr(m), rows, kn, _lib.ptr(ids), _lib.ptr(counts), _lib.stream(dev))
    return ids, counts


def density(dynamic_map: torch.Tensor, q_sizes: torch.Tensor, k_sizes: torch.Tensor) -> torch.Tensor:
    """map [..., Qc, Kc], sizes [..., Qc] / [..., Kc] -> kept-pair fraction [...] (fp32)."""
    dev = _lib.require_gpu(dynamic_map, q_sizes, k_sizes, what="density_calculation")
    qn, kn = dynamic_map.shape[-2:]
    lead = dynamic_map.shape[:-2]
    heads = int(torch.tensor(lead).prod().item()) if len(lead) else 1
    m = dynamic_map.to(torch.bool).contiguous()
    qs = q_sizes.to(torch.int32).reshape(heads, qn).contiguous()
    ks = k_sizes.to(torch.int32).reshape(heads, kn).contiguous()
    out = torch.empty(lead, dtype=torch.float32, device=dev)
    _lib.call("spr_density", _lib.ptr(m), _lib.ptr(qs), _lib.ptr(ks), heads, qn, kn, _lib.ptr(out),
              _lib.stream(dev))
    return out
