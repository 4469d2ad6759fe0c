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


PRECISION = {"high": 0, "highest": 1, "medium": 2}


def role_k_projection_normalize(k: torch.Tensor, k_factor: torch.Tensor, *, precision: str = "high",
                                weight: float = 1.0, out: torch.Tensor | None = None,
                                out_col: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Project K through its factor and divide by the head's RMS over (tokens, rank).

    The torch.compile'd ``_role_k_projection_normalize_fp32`` of n8_v6.py:141-149:
    key = bmm(k, k_factor) under the fp32 matmul precision (``"high"``: TF32 factor;
    ``"highest"``: fp32, as normalize_feature_scale(project_tokens(...)) computes it;
    ``"medium"``: bf16 factor), key_scale = sqrt(mean(key^2 over tokens and rank)).clamp_min(1e-8)
    per head; returns ((weight * key) / key_scale, key_scale [BH, 1, 1]).  With ``out`` the
    features go to columns out_col .. out_col + R of out [BH, N, C] (the K and weighted V halves
    of _role_kv_projection_normalize_fp32, n8_v6.py:91-103).  Two launches of the projection
    kernel (the first only sums p^2 per workgroup, deterministically, the second divides) so
    the fp32 key is written once.  bf16 K with D in {64, 128}, rank <= 128."""
    if k.ndim != 3 or k_factor.ndim != 3 or k_factor.shape[:2] != (k.shape[0], k.shape[2]):
        raise RuntimeError(f"Expected K[BH,N,D], F[BH,D,R], got {tuple(k.shape)}, {tuple(k_factor.shape)}.")
    if k.dtype != torch.bfloat16 or k.shape[2] not in (64, 128) or k_factor.shape[2] > 128:
        raise RuntimeError(f"The HIP K projection takes bf16 K with D in {{64, 128}} and R <= 128 "
                           f"(got {k.dtype}, D={k.shape[2]}, R={k_factor.shape[2]}).")
    if precision not in PRECISION:
        raise RuntimeError(f"role_kv_matmul_precision must be highest, high, or medium; got {precision!r}.")
    dev = _lib.require_gpu(k, k_factor, out, what="role K projection")
    bh, n, d = k.shape
    rank = int(k_factor.shape[2])
    kc = k.contiguous()
    f = k_factor.float().contiguous()
    if out is None:
        out = torch.empty((bh, n, rank), device=dev, dtype=torch.float32)
    elif (out.ndim != 3 or tuple(out.shape[:2]) != (bh, n) or out.dtype != torch.float32 or not out.is_contiguous()
          or out_col < 0 or out_col + rank > out.shape[2]):
        raise RuntimeError(f"K projection output must be contiguous fp32 [{bh}, {n}, >= {out_col + rank}], got "
                           f"{tuple(out.shape)} {out.dtype}.")
    scale = torch.empty((bh, 1, 1), device=dev, dtype=torch.float32)
    ws_bytes = int(_lib.query("spr_role_k_projection_workspace", bh, n))
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    _lib.call("spr_role_k_projection_ex", _lib.ptr(kc), _lib.ptr(f), bh, n, d, rank, PRECISION[precision],
              float(weight), _lib.ptr(out), int(out.shape[2]), int(out_col), _lib.ptr(scale), _lib.ptr(ws), ws.numel(),
              _lib.stream(dev))
    return out, scale


def role_kv_projection_normalize(k: torch.Tensor, v: torch.Tensor, k_factor: torch.Tensor, v_factor: torch.Tensor,
                                 v_weight: float, *, precision: str = "high"):
    """The joint K/V role features of ``_role_kv_projection_normalize_fp32`` (n8_v6.py:91-103):
    features [BH, N, R_k + R_v] = cat(key / key_scale, (v_weight value) / value_scale), each
    scale the RMS of its projection over the head.  Returns (features, key_scale, value_scale)."""
    bh, n = int(k.shape[0]), int(k.shape[1])
    rk, rv = int(k_factor.shape[2]), int(v_factor.shape[2])
    feats = torch.empty((bh, n, rk + rv), device=k.device, dtype=torch.float32)
    _, kscale = role_k_projection_normalize(k, k_factor, precision=precision, out=feats, out_col=0)
    _, vscale = role_k_projection_normalize(v, v_factor, precision=precision, weight=v_weight, out=feats,
                                            out_col=rk)
    return feats, kscale, vscale
