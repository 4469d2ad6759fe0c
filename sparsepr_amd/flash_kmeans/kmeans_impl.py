"""Batched Euclidean Lloyd iterations on the HIP kernels of csrc/spr_kmeans.hip.

One iteration is four launches and no host synchronisation (unless tol > 0):
  1. c_sq = ||c||^2 (fp32)                       spr_centroid_sq
  2. labels = argmin distance (bf16 MFMA)         spr_kmeans_assign_bf16
     or, for fp32 inputs, with the TF32 dot      spr_kmeans_assign_tf32
     products the reference's tl.dot forms
  3. stable counting sort of the labels           spr_argsort_labels
  4. segmented fp64 mean -> new centroids         spr_centroid_mean
The sort of step 3 in the last iteration is exactly argsort(final labels), so
the route reuses it as the cluster permutation.

Return convention (reference kmeans_triton_impl.py:102-115): labels from the
last assignment, centroids from the last update; when `shift < tol` stops the
loop, the centroids used by that last assignment are returned instead.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib

X_SQ_FP32 = 0  # inline fp32 squared norm (kmeans_utils.py:812-814)
X_SQ_BF16 = 1  # x.dtype buffer semantics of flash_kmeans (kmeans_triton_impl.py:84-87)


def _check_x(x: torch.Tensor, what: str):
    if x.dim() != 3:
        raise RuntimeError(f"{what} expects [B, N, D] input, got shape {tuple(x.shape)}.")
    return _lib.require_gpu(x, what=what)


def gather_rows(src: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """out[b, j] = src[b, idx[b, j]] for src [B, S, D], idx [B, M] (HIP gather)."""
    dev = _lib.require_gpu(src, idx, what="gather_rows")
    b, s, d = src.shape
    m = idx.shape[1]
    src_c = src.contiguous()
    ii = idx.to(torch.int32).contiguous()
    out = torch.empty((b, m, d), dtype=src.dtype, device=dev)
    _lib.call("spr_gather_rows", _lib.ptr(src_c), s, _lib.ptr(ii), _lib.ptr(out), m, b,
              d * src.element_size(), _lib.stream(dev))
    return out


def centroid_sq(c: torch.Tensor) -> torch.Tensor:
    dev = _lib.require_gpu(c, what="centroid_sq")
    if c.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"centroid_sq: unsupported dtype {c.dtype}")
    cc = c.contiguous()
    out = torch.empty(c.shape[:-1], dtype=torch.float32, device=dev)
    _lib.call("spr_centroid_sq", _lib.ptr(cc), _lib.DTYPE_CODE[c.dtype], cc.numel() // c.shape[-1],
              c.shape[-1], _lib.ptr(out), _lib.stream(dev))
    return out


def euclid_assign(x: torch.Tensor, centroids: torch.Tensor, x_sq: torch.Tensor | None = None,
                  *, x_sq_mode: int = X_SQ_BF16, c_sq: torch.Tensor | None = None,
                  out: torch.Tensor | None = None, x_sq_out: torch.Tensor | None = None) -> torch.Tensor:
    """Nearest-centroid ids int32 [B, N] (lowest index among exact minima).

    With x_sq None the squared norms are computed inline (per x_sq_mode); a float32
    [B, N] `x_sq_out` then receives them for reuse by later calls on the same x."""
    dev = _check_x(x, "euclid_assign")
    _lib.require_gpu(centroids, what="euclid_assign")
    B, N, D = x.shape
    K = centroids.shape[1]
    if centroids.shape != (B, K, D):
        raise RuntimeError("centroids shape mismatch")
    if centroids.dtype != x.dtype:
        raise RuntimeError("centroids dtype mismatch")
    if out is None:
        out = torch.empty((B, N), dtype=torch.int32, device=dev)
    xc = x.contiguous()
    cc = centroids.contiguous()
    if x.dtype == torch.bfloat16:
        if c_sq is None:
            c_sq = centroid_sq(cc)
        xs = None if x_sq is None else x_sq.to(torch.float32).contiguous()
        if x_sq_out is not None and (x_sq_out.shape != (B, N) or x_sq_out.dtype != torch.float32
                                     or not x_sq_out.is_contiguous()):
            raise RuntimeError("x_sq_out must be a contiguous float32 [B, N] tensor")
        _lib.call("spr_kmeans_assign_bf16", _lib.ptr(xc), _lib.ptr(cc), _lib.ptr(c_sq.contiguous()),
                  _lib.ptr(xs), int(x_sq_mode), _lib.ptr(x_sq_out if xs is None else None), B, N, K, D,
                  _lib.ptr(out), _lib.stream(dev))
    elif x.dtype == torch.float32:
        # tl.dot on fp32 operands rounds them to TF32 (assign_euclid_triton.py:897,
        # kmeans_utils.py:829); the products and the fp32 sums are otherwise exact
        if c_sq is None:
            c_sq = centroid_sq(cc)
        xs = None if x_sq is None else x_sq.to(torch.float32).contiguous()
        _lib.call("spr_kmeans_assign_tf32", _lib.ptr(xc), _lib.ptr(cc), _lib.ptr(c_sq.contiguous()), _lib.ptr(xs),
                  _lib.ptr(x_sq_out if xs is None else None), B, N, K, D, _lib.ptr(out), _lib.stream(dev))
    else:
        raise RuntimeError(f"euclid_assign: unsupported dtype {x.dtype} (bfloat16 or float32)")
    return out


@dataclass
class UpdateResult:
    centroids: torch.Tensor      # [B, K, D] x.dtype (bf16-rounded means)
    sizes: torch.Tensor          # int32 [B, K]
    sorted_idx: torch.Tensor     # int32 [B, N] stable argsort of the labels
    offsets: torch.Tensor        # int32 [B, K + 1] cluster start offsets in sorted order
    mean32: torch.Tensor | None  # fp32 means (before the cast to x.dtype)
    shift: torch.Tensor | None   # fp32 [1] max centroid movement


def centroid_update_sorted(x: torch.Tensor, labels: torch.Tensor, old: torch.Tensor, *,
                           want_mean32: bool = False, want_shift: bool = False,
                           sums_accum: torch.Tensor | None = None,
                           counts_accum: torch.Tensor | None = None,
                           sorted_idx=None, sizes=None, offsets=None, out: torch.Tensor | None = None,
                           c_sq_out: torch.Tensor | None = None) -> UpdateResult:
    """Cluster means of x under labels; empty clusters keep `old`."""
    dev = _check_x(x, "centroid_update")
    B, N, D = x.shape
    K = old.shape[1]
    if old.shape != (B, K, D):
        raise RuntimeError(f"old centroids must be {(B, K, D)}, got {tuple(old.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"centroid update: unsupported dtype {x.dtype}")
    if sorted_idx is None:
        from ..kernels.permute import argsort_labels

        sorted_idx, sizes, offsets = argsort_labels(labels.reshape(B, N), K)
    xc = x.contiguous()
    oc = old.to(x.dtype).contiguous()
    new = torch.empty_like(oc) if out is None else out
    mean32 = torch.empty((B, K, D), dtype=torch.float32, device=dev) if want_mean32 else None
    shift = torch.zeros(1, dtype=torch.float32, device=dev) if want_shift else None
    lib = _lib.load()
    ws_bytes = int(lib.spr_centroid_mean_workspace(B, N, K, D))
    ws = _lib.workspace(ws_bytes, dev) if ws_bytes > 0 else None
    _lib.call("spr_centroid_mean", _lib.ptr(xc), _lib.DTYPE_CODE[x.dtype], _lib.ptr(sorted_idx),
              _lib.ptr(offsets), _lib.ptr(oc), B, N, K, D, _lib.ptr(mean32), _lib.ptr(new),
              _lib.ptr(shift), _lib.ptr(sums_accum), _lib.ptr(counts_accum), _lib.ptr(c_sq_out), _lib.ptr(ws),
              ws_bytes, _lib.stream(dev))
    return UpdateResult(new, sizes, sorted_idx, offsets, mean32, shift)


@dataclass
class LloydResult:
    labels: torch.Tensor      # int32 [B, N]
    centroids: torch.Tensor   # [B, K, D] x.dtype
    sizes: torch.Tensor       # int32 [B, K] (counts of `labels`)
    iters: int
    sorted_idx: torch.Tensor  # int32 [B, N] stable argsort of `labels`
    offsets: torch.Tensor     # int32 [B, K + 1]
    mean32: torch.Tensor | None = None


def random_init(x: torch.Tensor, n_clusters: int, generator=None) -> torch.Tensor:
    """Initial centroids = x rows at uniform random indices (kmeans_triton_impl.py:89-96)."""
    B, N, _ = x.shape
    idx = torch.randint(0, N, (B, n_clusters), device=x.device, generator=generator, dtype=torch.int64)
    return gather_rows(x, idx.to(torch.int32))


def lloyd(x: torch.Tensor, n_clusters: int, max_iters: int, tol: float = 0.0,
          init_centroids: torch.Tensor | None = None, *, x_sq: torch.Tensor | None = None,
          x_sq_mode: int = X_SQ_BF16, verbose: bool = False, want_mean32: bool = False) -> LloydResult:
    """Batched Lloyd loop; see the module docstring for the return convention."""
    dev = _check_x(x, "batch_kmeans_Euclid")
    if max_iters < 1:
        raise RuntimeError("lloyd requires max_iters >= 1")
    B, N, D = x.shape
    K = int(n_clusters)
    x = x.contiguous()
    if init_centroids is None:
        cent = random_init(x, K)
    else:
        cent = init_centroids.reshape(B, K, D).to(x.dtype).contiguous()
    from ..kernels.permute import argsort_labels

    labels = torch.empty((B, N), dtype=torch.int32, device=dev)
    # squared point norms: computed by the first assignment, reused afterwards
    cached_sq = None
    if x_sq is None and max_iters > 1:
        cached_sq = torch.empty((B, N), dtype=torch.float32, device=dev)
    res = None
    it = -1
    # centroid norms: computed once, then produced by each update for the next assignment
    c_sq = centroid_sq(cent)
    for it in range(max_iters):
        if x_sq is None and cached_sq is not None and it > 0:
            euclid_assign(x, cent, cached_sq, x_sq_mode=x_sq_mode, c_sq=c_sq, out=labels)
        else:
            euclid_assign(x, cent, x_sq, x_sq_mode=x_sq_mode, c_sq=c_sq, out=labels, x_sq_out=cached_sq)
        sorted_idx, sizes, offsets = argsort_labels(labels, K)
        next_sq = torch.empty((B, K), dtype=torch.float32, device=dev) if c_sq is not None else None
        res = centroid_update_sorted(x, labels, cent, want_mean32=want_mean32, want_shift=tol > 0 or verbose,
                                     sorted_idx=sorted_idx, sizes=sizes, offsets=offsets, c_sq_out=next_sq)
        c_sq = next_sq
        if verbose:
            print(f"Iter {it}, center shift: {float(res.shift.item()):.6f}")
        if tol > 0 and float(res.shift.item()) < tol:
            return LloydResult(labels, cent, sizes, it + 1, sorted_idx, offsets, res.mean32)
        cent = res.centroids
    return LloydResult(labels, cent, res.sizes, it + 1, res.sorted_idx, res.offsets, res.mean32)
