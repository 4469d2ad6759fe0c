"""Drop-in for src/sparsepr/kernels/triton/rrr_eigensolver.py: the fixed-count top-16
subspace basis of the N8 repair's 64 x 128 weighted residual, on spr_rrr_top16_basis
(csrc/spr_rrr.hip rrr_top16_kernel, one workgroup per head)."""

from __future__ import annotations

import torch

from .. import _lib


def top16_right_basis_triton(weighted_fitted: torch.Tensor, *, power_iters: int = 8,
                             inv_sqrt_iters: int = 6) -> torch.Tensor:
    """Approximate the top-16 right singular subspace of [BH, 64, 128] (reference :86-128):
    power_iters subspace steps on the 64 x 64 row Gram from the cosine seed, each
    orthonormalised by inv_sqrt_iters Newton-Schulz steps, then V^T Q orthonormalised the
    same way.  Returns fp32 [BH, 128, 16]."""
    if not weighted_fitted.is_cuda:
        raise RuntimeError("top16_right_basis_triton requires CUDA tensors.")
    if tuple(weighted_fitted.shape[1:]) != (64, 128):
        raise RuntimeError(f"N8 top-16 kernel requires [BH,64,128], got {tuple(weighted_fitted.shape)}.")
    if power_iters <= 0 or inv_sqrt_iters <= 0:
        raise RuntimeError("Subspace iteration counts must be positive.")
    dev = _lib.require_gpu(weighted_fitted, what="top-16 subspace basis")
    values = weighted_fitted.float().contiguous()
    bh = int(values.shape[0])
    basis = torch.empty((bh, 128, 16), device=dev, dtype=torch.float32)
    _lib.call("spr_rrr_top16_basis", _lib.ptr(values), bh, int(power_iters), int(inv_sqrt_iters), _lib.ptr(basis),
              _lib.stream(dev))
    return basis
