"""Cluster permutation of [B, H, S, D] tensors along the sequence axis.

Drop-in for the reference's src/sparsepr/kernels/triton/permute.py: same
function names, arguments, return values and errors.  The gather / scatter runs
in the HIP kernels of csrc/spr_permute.hip; `argsort(labels)` is the stable
counting sort of csrc/spr_sort.hip (ties keep ascending token order).
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _lib


def argsort_labels(labels: torch.Tensor, num_clusters: int | None = None):
    """Stable per-row argsort of integer cluster labels [R, S].

    Returns (sorted_indices int32 [R, S], sizes int32 [R, K], offsets int32 [R, K+1]).
    `num_clusters` defaults to labels.max() + 1 (one device->host read)."""
    dev = _lib.require_gpu(labels, what="argsort_labels")
    if labels.dim() != 2:
        raise RuntimeError(f"argsort_labels expects [R, S] labels, got {tuple(labels.shape)}")
    lab = labels if labels.dtype == torch.int32 else labels.to(torch.int32)
    lab = lab.contiguous()
    rows, n = lab.shape
    if num_clusters is None:
        num_clusters = int(lab.max().item()) + 1 if lab.numel() else 1
    k = int(num_clusters)
    idx = torch.empty((rows, n), dtype=torch.int32, device=dev)
    sizes = torch.empty((rows, k), dtype=torch.int32, device=dev)
    offsets = torch.empty((rows, k + 1), dtype=torch.int32, device=dev)
    ws_bytes = _lib.query("spr_argsort_labels_workspace", rows, n, k)
    ws = _lib.workspace(ws_bytes, dev)
    _lib.call("spr_argsort_labels", _lib.ptr(lab), rows, n, k, _lib.ptr(idx), _lib.ptr(sizes),
              _lib.ptr(offsets), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
    return idx, sizes, offsets


def _sorted_indices_for(labels, sorted_indices, bh, s, device, num_clusters=None):
    if sorted_indices is not None:
        si = sorted_indices.to(device=device, dtype=torch.int32).reshape(bh, s).contiguous()
        return si
    if labels is None:
        raise AssertionError("Either `labels` or `sorted_indices` must be provided.")
    lab = labels.to(device).reshape(bh, s)
    return argsort_labels(lab, num_clusters)[0]


def permute_tensor_by_labels_triton(
    tensor: torch.Tensor,
    labels: Optional[torch.Tensor],
    dim: int,
    *,
    sorted_indices: Optional[torch.Tensor] = None,
    num_clusters: int | None = None,
):
    """Permute `tensor` [B,H,S,D] along dim 2 into ascending label order.

    Reference: permute.py:126-172.  Returns (permuted, sorted_indices int32 [B*H, S])."""
    assert dim == 2, "permute_tensor_by_labels currently only supports dim==2 (sequence dimension)"
    assert tensor.dim() == 4, "Expected tensor shape [B,H,S,D]"
    dev = _lib.require_gpu(tensor, what="permute_tensor_by_labels")
    B, H, S, D = tensor.shape
    bh = B * H
    si = _sorted_indices_for(labels, sorted_indices, bh, S, dev, num_clusters)
    inp = tensor.reshape(bh, S, D).contiguous()
    out = torch.empty_like(inp)
    _lib.call("spr_permute_rows", _lib.ptr(inp), _lib.ptr(si), _lib.ptr(out), bh, S,
              D * inp.element_size(), _lib.stream(dev))
    return out.reshape(B, H, S, D), si


def permute_concatenated_tensors_by_labels_triton(
    prefix: torch.Tensor,
    suffix: torch.Tensor,
    labels: Optional[torch.Tensor],
    dim: int,
    *,
    sorted_indices: Optional[torch.Tensor] = None,
):
    """Permute cat((prefix, suffix), dim=2) without materialising the cat.

    Reference: permute.py:175-232 (same shape checks and errors)."""
    assert dim == 2, "concatenated permutation only supports dim==2"
    assert prefix.dim() == 4 and suffix.dim() == 4, "Expected [B,H,S,D] inputs"
    dev = _lib.require_gpu(prefix, suffix, what="concatenated permutation")
    if prefix.shape[:2] != suffix.shape[:2] or prefix.shape[3] != suffix.shape[3]:
        raise RuntimeError(
            "Concatenated permutation shape mismatch: "
            f"prefix={tuple(prefix.shape)}, suffix={tuple(suffix.shape)}."
        )
    if prefix.dtype != suffix.dtype or prefix.device != suffix.device:
        raise RuntimeError("Concatenated permutation inputs must share dtype and device.")
    batch, heads, prefix_s, dim_size = prefix.shape
    suffix_s = int(suffix.shape[2])
    total_s = prefix_s + suffix_s
    bh = batch * heads
    if sorted_indices is None:
        if labels is None:
            raise RuntimeError("Either labels or sorted_indices must be provided.")
        if tuple(labels.shape) != (bh, total_s):
            raise RuntimeError(f"Label shape {tuple(labels.shape)} does not match {(bh, total_s)}.")
        si = argsort_labels(labels.to(dev))[0]
    else:
        if tuple(sorted_indices.shape) != (bh, total_s):
            raise RuntimeError(
                f"Sorted-index shape {tuple(sorted_indices.shape)} does not match {(bh, total_s)}."
            )
        si = sorted_indices.to(torch.int32).contiguous()
    pre = prefix.reshape(bh, prefix_s, dim_size).contiguous()
    suf = suffix.reshape(bh, suffix_s, dim_size).contiguous()
    out = torch.empty((bh, total_s, dim_size), device=dev, dtype=prefix.dtype)
    _lib.call("spr_permute_concat_rows", _lib.ptr(pre), _lib.ptr(suf), _lib.ptr(si), _lib.ptr(out), bh,
              prefix_s, suffix_s, dim_size * pre.element_size(), _lib.stream(dev))
    return out.view(batch, heads, total_s, dim_size), si


def apply_inverse_permutation_triton(
    permuted_tensor: torch.Tensor,
    sorted_indices: torch.Tensor,
    dim: int,
):
    """Undo permute_tensor_by_labels_triton: out[b, idx[b, s]] = in[b, s].

    Reference: permute.py:235-274."""
    assert dim == 2, "apply_inverse_permutation currently only supports dim==2"
    assert permuted_tensor.dim() == 4, "Expected tensor shape [B,H,S,D]"
    dev = _lib.require_gpu(permuted_tensor, sorted_indices, what="apply_inverse_permutation")
    B, H, S, D = permuted_tensor.shape
    bh = B * H
    si = sorted_indices.to(torch.int32).reshape(bh, S).contiguous()
    t = permuted_tensor
    # rows packed within each head and one stride of at least S rows between heads (a slice
    # of the rows of a longer tensor, e.g. the video part of an attention output): read in
    # place.  Anything else (an expanded tensor's zero head stride included) is copied first.
    head = t.stride(1) if H > 1 else (t.stride(0) if B > 1 else S * D)
    if (t.stride(3) == 1 and t.stride(2) == D and (H == 1 or t.stride(0) == H * t.stride(1))
            and head >= S * D):
        out = torch.empty((bh, S, D), dtype=t.dtype, device=dev)
        _lib.call("spr_inverse_permute_rows_strided", _lib.ptr(t), head * t.element_size(), _lib.ptr(si),
                  _lib.ptr(out), bh, S, D * t.element_size(), _lib.stream(dev))
        return out.reshape(B, H, S, D)
    inp = t.reshape(bh, S, D).contiguous()
    out = torch.empty_like(inp)
    _lib.call("spr_inverse_permute_rows", _lib.ptr(inp), _lib.ptr(si), _lib.ptr(out), bh, S,
              D * inp.element_size(), _lib.stream(dev))
    return out.reshape(B, H, S, D)


# Names used by call sites that import the pure-torch references
# (kmeans_utils.py:1674-1695); same results, HIP kernels underneath.
def permute_tensor_by_labels(tensor, labels, dim):
    return permute_tensor_by_labels_triton(tensor, labels, dim)


def apply_inverse_permutation(permuted_tensor, sorted_indices, dim):
    return apply_inverse_permutation_triton(permuted_tensor, sorted_indices, dim)
