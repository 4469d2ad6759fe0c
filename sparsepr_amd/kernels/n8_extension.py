"""Native N8 kernels (drop-in for the reference's src/sparsepr/kernels/n8_extension.py).

The reference loads a pybind module `n8_kernels` built from n8_ops.cu.  Here the
same entry points are served by libsparsepr_hip.so through its C ABI.
`load_n8_kernels()` returns a module-like object exposing the reference's export
names (n8_ops.cu:642-664) so `hasattr` capability probes keep working.
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


def _qkv_common(q, k, v, what):
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError(f"{what} QKV inputs must be CUDA tensors")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise RuntimeError(f"{what} QKV inputs must be contiguous")
    if q.shape != k.shape or q.shape != v.shape or q.dim() != 3:
        raise RuntimeError(f"{what} QKV inputs must have matching [B,{'L' if what == 'Wan' else 'S'},C] shapes")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise RuntimeError(f"{what} QKV dtypes must match")
    if q.dtype not in _lib.DTYPE_CODE:
        raise RuntimeError(f"{what} QKV dtype {q.dtype} is not bf16, fp16 or fp32")


def wan_qkv_norm_rope_layout(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                             k_weight: torch.Tensor, freq_real: torch.Tensor, freq_imag: torch.Tensor, *,
                             heads: int, epsilon: float):
    """Native-Wan Q/K RMSNorm over all C channels, complex-pair RoPE and the BHLD layout
    (n8_ops.cu:16-105, host :356-413): q, k, v [B, L, C] -> three [B, H, L, D] tensors."""
    _qkv_common(q, k, v, "Wan")
    if not (q_weight.is_cuda and k_weight.is_cuda and q_weight.is_contiguous() and k_weight.is_contiguous()):
        raise RuntimeError("Wan norm weights must be contiguous CUDA tensors")
    if q_weight.dtype != q.dtype or k_weight.dtype != q.dtype:
        raise RuntimeError("Wan norm weights must match the QKV dtype")
    if not (freq_real.is_cuda and freq_imag.is_cuda and freq_real.dtype == torch.float32
            and freq_imag.dtype == torch.float32 and freq_real.is_contiguous() and freq_imag.is_contiguous()):
        raise RuntimeError("Wan RoPE frequency tensors must be contiguous CUDA FP32")
    batch, tokens, channels = (int(x) for x in q.shape)
    heads = int(heads)
    if heads <= 0 or channels % heads != 0:
        raise RuntimeError("Wan channels must divide num_heads")
    head_dim = channels // heads
    if head_dim % 2 != 0:
        raise RuntimeError("Wan head_dim must be even")
    if q_weight.numel() != channels or k_weight.numel() != channels:
        raise RuntimeError("Wan norm weights must contain C elements")
    if (freq_real.shape != freq_imag.shape or freq_real.dim() != 2 or freq_real.shape[0] != tokens
            or freq_real.shape[1] != head_dim // 2):
        raise RuntimeError("Wan RoPE frequencies must have shape [L,D/2]")
    dev = _lib.require_gpu(q, k, v, q_weight, k_weight, freq_real, freq_imag, what="Wan QKV")
    out = [torch.empty((batch, heads, tokens, head_dim), dtype=q.dtype, device=dev) for _ in range(3)]
    _lib.call("spr_wan_qkv_norm_rope_layout", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(q_weight),
              _lib.ptr(k_weight), _lib.ptr(freq_real), _lib.ptr(freq_imag), _lib.DTYPE_CODE[q.dtype], batch, tokens,
              channels, heads, float(epsilon), *[_lib.ptr(t) for t in out], _lib.stream(dev))
    return tuple(out)


def cosmos25_qkv_norm_rope_bshd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                                k_weight: torch.Tensor, rope_angles: torch.Tensor, *, heads: int, epsilon: float):
    """Cosmos2.5 per-head Q/K RMSNorm (fp32 weights) and Transformer-Engine rotate-half RoPE
    (n8_ops.cu:107-187, host :415-497): q, k, v [B, S, H*D] -> three [B, S, H, D] tensors."""
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    _qkv_common(q, k, v, "Cosmos2.5")
    q_weight = q_weight.float().contiguous()
    k_weight = k_weight.float().contiguous()
    rope_angles = rope_angles.float().contiguous()
    if not (q_weight.is_cuda and k_weight.is_cuda):
        raise RuntimeError("Cosmos2.5 norm weights must be contiguous CUDA FP32 tensors")
    if not rope_angles.is_cuda:
        raise RuntimeError("Cosmos2.5 RoPE angles must be contiguous CUDA FP32")
    if len({t.device for t in (q, k, v, q_weight, k_weight, rope_angles)}) != 1:
        raise RuntimeError("Cosmos2.5 QKV, weights, and RoPE angles must share one CUDA device")
    batch, tokens, channels = (int(x) for x in q.shape)
    heads = int(heads)
    if heads <= 0 or channels % heads != 0:
        raise RuntimeError("Cosmos2.5 channels must divide num_heads")
    head_dim = channels // heads
    if head_dim <= 0 or head_dim % 2 != 0:
        raise RuntimeError("Cosmos2.5 head_dim must be positive and even")
    if q_weight.numel() != head_dim or k_weight.numel() != head_dim:
        raise RuntimeError("Cosmos2.5 norm weights must contain head_dim elements")
    if tuple(rope_angles.shape) != (tokens, 1, 1, head_dim):
        raise RuntimeError("Cosmos2.5 RoPE angles must have shape [S,1,1,D]")
    if not epsilon > 0.0:
        raise RuntimeError("Cosmos2.5 RMSNorm epsilon must be positive")
    dev = q.device
    out = [torch.empty((batch, tokens, heads, head_dim), dtype=q.dtype, device=dev) for _ in range(3)]
    _lib.call("spr_cosmos25_qkv_norm_rope_bshd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(q_weight),
              _lib.ptr(k_weight), _lib.ptr(rope_angles), _lib.DTYPE_CODE[q.dtype], batch, tokens, heads, head_dim,
              float(epsilon), *[_lib.ptr(t) for t in out], _lib.stream(dev))
    return tuple(out)


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
        "wan_qkv_norm_rope_layout": lambda q, k, v, qw, kw, fr, fi, heads, eps: list(
            wan_qkv_norm_rope_layout(q, k, v, qw, kw, fr, fi, heads=heads, epsilon=eps)),
        "cosmos25_qkv_norm_rope_bshd": lambda q, k, v, qw, kw, ang, heads, eps: list(
            cosmos25_qkv_norm_rope_bshd(q, k, v, qw, kw, ang, heads=heads, epsilon=eps)),
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
