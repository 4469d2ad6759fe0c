"""Role-coordinate projection + row RMS normalisation on the HIP kernel of
csrc/spr_role_proj.hip.

Same name, keyword signature, validation and error texts as the reference's
src/sparsepr/kernels/triton/role_projection.py:58-103 (role_projection_rms_triton).
block_m and num_warps are validated as the reference validates them and otherwise
ignored (the HIP kernel has one tiling).  The HIP path takes bf16 X (the model's
activations, which the reference promotes to fp32 exactly) with D in {64, 128} and
R <= 128; other inputs raise.  The factor is rounded to TF32 as the reference's
tl.dot(..., input_precision="tf32") does.  There is no CPU path.
"""

from __future__ import annotations

import torch

from .. import _lib


def role_projection_rms_triton(
    x: torch.Tensor,
    factor: torch.Tensor,
    *,
    block_m: int = 16,
    num_warps: int = 4,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Project ``[BH,N,D]`` through ``[BH,D,R]`` and RMS-normalize rows."""
    if not x.is_cuda or not factor.is_cuda:
        raise RuntimeError("Role projection requires CUDA tensors.")
    if x.ndim != 3 or factor.ndim != 3:
        raise RuntimeError(f"Expected X[BH,N,D], F[BH,D,R], got {x.shape}, {factor.shape}.")
    bh, tokens, dim = x.shape
    if factor.shape[0] != bh or factor.shape[1] != dim:
        raise RuntimeError(f"Role projection shape mismatch: X={x.shape}, F={factor.shape}.")
    rank = int(factor.shape[2])
    if dim > 256 or rank > 128:
        raise RuntimeError("Fused role projection currently supports D<=256 and R<=128.")
    if block_m not in {16, 32, 64}:
        raise RuntimeError("Role projection tensor-core BLOCK_M must be one of 16,32,64.")
    if num_warps not in {2, 4, 8}:
        raise RuntimeError("Role projection num_warps must be one of 2,4,8.")
    if x.dtype != torch.bfloat16 or dim not in (64, 128):
        raise RuntimeError(f"The HIP role projection takes bf16 X with D in {{64, 128}} (got {x.dtype}, D={dim}).")
    dev = _lib.require_gpu(x, factor, out, what="role projection")
    x = x.contiguous()
    factor = factor.float().contiguous()
    if out is None:
        out = torch.empty((bh, tokens, rank), device=x.device, dtype=torch.float32)
    elif out.shape != (bh, tokens, rank) or out.device != x.device or out.dtype != torch.float32:
        raise RuntimeError(
            f"Role projection output must be {(bh, tokens, rank)} FP32 on {x.device}, got "
            f"{tuple(out.shape)} {out.dtype} {out.device}."
        )
    elif not out.is_contiguous():
        raise RuntimeError("Role projection output must be contiguous.")
    _lib.call("spr_role_projection_rms", _lib.ptr(x), _lib.ptr(factor), bh, tokens, dim, rank, _lib.ptr(out),
              _lib.stream(dev))
    return out


def role_k_projection_normalize(k: torch.Tensor, k_factor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Project K through its factor and divide by the head's RMS over (tokens, rank).

    The torch.compile'd ``_role_k_projection_normalize_fp32`` of n8_v6.py:141-149:
    key = bmm(k, k_factor) (TF32 factor, as the reference's fp32 matmul under its TF32
    contract), key_scale = sqrt(mean(key^2 over tokens and rank)).clamp_min(1e-8) per head,
    returns (key / key_scale, key_scale [BH, 1, 1]).  Two launches of the projection kernel
    (the first only sums p^2 per workgroup, deterministically, the second divides) so the
    fp32 key is written once.  bf16 K with D in {64, 128}, rank <= 128."""
    if k.ndim != 3 or k_factor.ndim != 3 or k_factor.shape[:2] != (k.shape[0], k.shape[2]):
        raise RuntimeError(f"Expected K[BH,N,D], F[BH,D,R], got {tuple(k.shape)}, {tuple(k_factor.shape)}.")
    if k.dtype != torch.bfloat16 or k.shape[2] not in (64, 128) or k_factor.shape[2] > 128:
        raise RuntimeError(f"The HIP K projection takes bf16 K with D in {{64, 128}} and R <= 128 "
                           f"(got {k.dtype}, D={k.shape[2]}, R={k_factor.shape[2]}).")
    dev = _lib.require_gpu(k, k_factor, what="role K projection")
    bh, n, d = k.shape
    rank = int(k_factor.shape[2])
    kc = k.contiguous()
    f = k_factor.float().contiguous()
    out = torch.empty((bh, n, rank), device=dev, dtype=torch.float32)
    scale = torch.empty((bh, 1, 1), device=dev, dtype=torch.float32)
    ws_bytes = int(_lib.query("spr_role_k_projection_workspace", bh, n))
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    _lib.call("spr_role_k_projection", _lib.ptr(kc), _lib.ptr(f), bh, n, d, rank, _lib.ptr(out), _lib.ptr(scale),
              _lib.ptr(ws), ws.numel(), _lib.stream(dev))
    return out, scale
