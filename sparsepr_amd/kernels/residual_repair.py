"""Repair epilogues (drop-in for the reference's src/sparsepr/kernels/triton/residual_repair.py:
the output-only and the output + role feature paths) on the HIP kernels of csrc/spr_repair.hip."""

from __future__ import annotations

import torch

from .. import _lib


def n8_prepare_output_repair_fit_triton(base, dense_probes, rows, x_fit, dense_float, y_fit, *, block_m=16):
    """x_fit = float(base[rows]), dense_float = float(dense), y_fit = dense - x_fit
    (reference residual_repair.py:798-857; same shape/device checks)."""
    del block_m
    bh, tokens, base_dim = base.shape
    probes = int(rows.shape[1])
    expected = {
        "dense": (bh, probes, base_dim), "rows": (bh, probes), "x_fit": (bh, probes, base_dim),
        "dense_float": (bh, probes, base_dim), "y_fit": (bh, probes, base_dim),
    }
    actual = {
        "dense": tuple(dense_probes.shape), "rows": tuple(rows.shape), "x_fit": tuple(x_fit.shape),
        "dense_float": tuple(dense_float.shape), "y_fit": tuple(y_fit.shape),
    }
    mismatched = {k: (actual[k], v) for k, v in expected.items() if actual[k] != v}
    if mismatched:
        raise RuntimeError(f"Invalid output-only fit-preparation shapes: {mismatched}.")
    if not base.is_cuda or any(t.device != base.device for t in (dense_probes, rows, x_fit, dense_float, y_fit)):
        raise RuntimeError("Output-only fit preparation requires one CUDA device.")
    if any(not t.is_contiguous() for t in (base, dense_probes, x_fit, dense_float, y_fit)):
        raise RuntimeError("Output-only fit preparation requires contiguous tensors.")
    if any(t.dtype != torch.float32 for t in (x_fit, dense_float, y_fit)):
        raise RuntimeError("Output-only fit preparation writes fp32 buffers.")
    rows_i32 = rows.to(torch.int32).contiguous()
    _lib.call("spr_repair_fit_prep", _lib.ptr(base), _lib.DTYPE_CODE[base.dtype], _lib.ptr(dense_probes),
              _lib.DTYPE_CODE[dense_probes.dtype], _lib.ptr(rows_i32), bh, tokens, probes, base_dim,
              _lib.ptr(x_fit), _lib.ptr(dense_float), _lib.ptr(y_fit), _lib.stream(base.device))
    return x_fit, dense_float, y_fit


def n8_prepare_repair_fit_triton(base, role, dense_probes, rows, x_fit, dense_float, y_fit, *, block_m=16):
    """x_fit = [float(base[rows]), float(role[rows])], dense_float = float(dense), y_fit =
    dense - float(base[rows]) (reference residual_repair.py:737-797; same shape/device
    checks).  role fp32 [BH, N, R]."""
    del block_m
    bh, tokens, base_dim = base.shape
    role_dim = int(role.shape[2])
    probes = int(rows.shape[1])
    expected = {
        "role": (bh, tokens, role_dim), "dense": (bh, probes, base_dim), "rows": (bh, probes),
        "x_fit": (bh, probes, base_dim + role_dim), "dense_float": (bh, probes, base_dim),
        "y_fit": (bh, probes, base_dim),
    }
    actual = {
        "role": tuple(role.shape), "dense": tuple(dense_probes.shape), "rows": tuple(rows.shape),
        "x_fit": tuple(x_fit.shape), "dense_float": tuple(dense_float.shape), "y_fit": tuple(y_fit.shape),
    }
    mismatched = {k: (actual[k], v) for k, v in expected.items() if actual[k] != v}
    if mismatched:
        raise RuntimeError(f"Invalid fused fit-preparation shapes: {mismatched}.")
    if not base.is_cuda or any(t.device != base.device for t in (role, dense_probes, rows, x_fit, dense_float, y_fit)):
        raise RuntimeError("Fused fit preparation requires one CUDA device.")
    if any(not t.is_contiguous() for t in (base, role, dense_probes, x_fit, dense_float, y_fit)):
        raise RuntimeError("Fused fit preparation requires contiguous tensors.")
    if any(t.dtype != torch.float32 for t in (role, x_fit, dense_float, y_fit)):
        raise RuntimeError("Fused fit preparation takes fp32 role features and writes fp32 buffers.")
    rows_i32 = rows.to(torch.int32).contiguous()
    _lib.call("spr_repair_fit_prep_role", _lib.ptr(base), _lib.DTYPE_CODE[base.dtype], _lib.ptr(role), role_dim,
              _lib.ptr(dense_probes), _lib.DTYPE_CODE[dense_probes.dtype], _lib.ptr(rows_i32), bh, tokens, probes,
              base_dim, _lib.ptr(x_fit), _lib.ptr(dense_float), _lib.ptr(y_fit), _lib.stream(base.device))
    return x_fit, dense_float, y_fit


def n8_repair_apply_triton(base, role, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, *, block_n=16,
                           num_warps=4, num_stages=2, input_precision="ieee", out=None):
    """base + alpha * ((((base, role) - mu) / sigma) left basis^T + y_mean) with an optional
    norm cap on the base norm, fixed D=128, role 64, rank 16 (reference
    residual_repair.py:388-475, kernel :10-92)."""
    if not base.is_cuda:
        raise RuntimeError("n8_repair_apply_triton requires CUDA tensors.")
    bh, tokens, base_dim = base.shape
    role_dim = int(role.shape[2])
    rank = int(left.shape[2])
    if (base_dim, role_dim, rank) != (128, 64, 16):
        raise RuntimeError(
            "The specialized N8 repair kernel requires D=128, role=64, rank=16; "
            f"got D={base_dim}, role={role_dim}, rank={rank}."
        )
    expected = {"role": (bh, tokens, role_dim), "x_mean": (bh, 1, base_dim + role_dim),
                "x_scale": (bh, 1, base_dim + role_dim), "y_mean": (bh, 1, base_dim),
                "left": (bh, base_dim + role_dim, rank), "basis": (bh, base_dim, rank)}
    actual = {"role": tuple(role.shape), "x_mean": tuple(x_mean.shape), "x_scale": tuple(x_scale.shape),
              "y_mean": tuple(y_mean.shape), "left": tuple(left.shape), "basis": tuple(basis.shape)}
    mismatched = {k: (actual[k], v) for k, v in expected.items() if actual[k] != v}
    if mismatched:
        raise RuntimeError(f"Invalid specialized N8 repair shapes: {mismatched}.")
    if any(not t.is_contiguous() for t in (base, role, x_mean, x_scale, y_mean, left, basis)):
        raise RuntimeError("The specialized N8 repair kernel requires contiguous tensors.")
    if block_n not in {8, 16, 32, 64}:
        raise RuntimeError(f"N8 repair BLOCK_N must be one of 8,16,32,64, got {block_n}.")
    if num_warps not in {2, 4, 8}:
        raise RuntimeError(f"N8 repair num_warps must be one of 2,4,8, got {num_warps}.")
    if num_stages not in {1, 2, 3, 4}:
        raise RuntimeError("N8 repair num_stages must be one of 1,2,3,4.")
    if input_precision not in {"ieee", "tf32"}:
        raise RuntimeError("N8 repair input_precision must be 'ieee' or 'tf32'.")
    if base.dtype != torch.bfloat16:
        raise RuntimeError("The specialized N8 repair kernel requires bfloat16 base rows.")
    if out is None:
        out = torch.empty_like(base)
    elif tuple(out.shape) != tuple(base.shape) or out.device != base.device or out.dtype != base.dtype:
        raise RuntimeError(f"N8 repair output must match base, got {tuple(out.shape)} {out.dtype} {out.device}.")
    elif not out.is_contiguous():
        raise RuntimeError("N8 repair output must be contiguous.")
    return repair_apply_role(base, role, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, out=out)


def repair_apply_role(base, role, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, out=None):
    """The apply kernel with role features: bf16 base [BH, N, D], D in {64, 128}; role fp32
    [BH, N, R], R in {16, 32, 48, 64}; rank 16, 32 or 64; x_mean / x_scale hold D + R
    entries."""
    bh, tokens, dim = base.shape
    role_dim = int(role.shape[2])
    rank = int(left.shape[2])
    if dim not in (64, 128) or rank not in (16, 32, 64) or base.dtype != torch.bfloat16 or role_dim not in (16, 32, 48, 64):
        raise RuntimeError(f"repair apply kernel needs bf16 D in (64, 128), role in (16, 32, 48, 64) and rank in "
                           f"(16, 32, 64); "
                           f"got {base.dtype} D={dim} role={role_dim} r={rank}")
    if out is None:
        out = torch.empty_like(base)
    rf = role.float().contiguous()
    f = [t.float().contiguous() for t in (x_mean, x_scale, y_mean, left, basis)]
    _lib.call("spr_repair_apply_role", _lib.ptr(base), _lib.ptr(rf), role_dim, *[_lib.ptr(t) for t in f], bh, tokens,
              dim, rank, float(alpha), float(norm_cap), _lib.ptr(out), _lib.stream(base.device))
    return out


def n8_repair_apply_output_triton(base, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, *, block_n=16,
                                  num_warps=4, num_stages=2, input_precision="ieee", out=None):
    """base + alpha * (((base - mu) / sigma) left basis^T + y_mean) with an optional
    norm cap, fixed D=128, rank=16 (reference residual_repair.py:478-562)."""
    del block_n, num_warps, num_stages
    if not base.is_cuda:
        raise RuntimeError("n8_repair_apply_output_triton requires CUDA tensors.")
    bh, tokens, base_dim = base.shape
    rank = int(left.shape[2])
    if (base_dim, rank) != (128, 16):
        raise RuntimeError(
            "The output-only N8 repair kernel requires D=128, rank=16; "
            f"got D={base_dim}, rank={rank}."
        )
    expected = {"x_mean": (bh, 1, base_dim), "x_scale": (bh, 1, base_dim), "y_mean": (bh, 1, base_dim),
                "left": (bh, base_dim, rank), "basis": (bh, base_dim, rank)}
    actual = {"x_mean": tuple(x_mean.shape), "x_scale": tuple(x_scale.shape), "y_mean": tuple(y_mean.shape),
              "left": tuple(left.shape), "basis": tuple(basis.shape)}
    mismatched = {k: (actual[k], v) for k, v in expected.items() if actual[k] != v}
    if mismatched:
        raise RuntimeError(f"Invalid output-only N8 repair shapes: {mismatched}.")
    tensors = (base, x_mean, x_scale, y_mean, left, basis)
    if any(not t.is_contiguous() for t in tensors):
        raise RuntimeError("The output-only N8 repair kernel requires contiguous tensors.")
    if input_precision not in {"ieee", "tf32"}:
        raise RuntimeError("N8 repair input_precision must be 'ieee' or 'tf32'.")
    if base.dtype != torch.bfloat16:
        raise RuntimeError("The output-only N8 repair kernel requires bfloat16 base rows.")
    if out is None:
        out = torch.empty_like(base)
    elif tuple(out.shape) != tuple(base.shape) or out.device != base.device or out.dtype != base.dtype:
        raise RuntimeError(f"N8 repair output must match base, got {tuple(out.shape)} {out.dtype} {out.device}.")
    elif not out.is_contiguous():
        raise RuntimeError("N8 repair output must be contiguous.")
    f = [t.float().contiguous() for t in (x_mean, x_scale, y_mean, left, basis)]
    _lib.call("spr_repair_apply", _lib.ptr(base), *[_lib.ptr(t) for t in f], bh, tokens, base_dim, rank,
              float(alpha), float(norm_cap), _lib.ptr(out), _lib.stream(base.device))
    return out


def repair_apply_output(base, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, out=None):
    """The apply kernel for bf16 base [BH, N, D], D in {64, 128}, rank 16, 32 or 64."""
    bh, tokens, dim = base.shape
    rank = int(left.shape[2])
    if dim not in (64, 128) or rank not in (16, 32, 64) or base.dtype != torch.bfloat16:
        raise RuntimeError(f"repair apply kernel needs bf16 D in (64, 128) and rank in (16, 32, 64); got {base.dtype} "
                           f"D={dim} r={rank}")
    if out is None:
        out = torch.empty_like(base)
    f = [t.float().contiguous() for t in (x_mean, x_scale, y_mean, left, basis)]
    _lib.call("spr_repair_apply", _lib.ptr(base), *[_lib.ptr(t) for t in f], bh, tokens, dim, rank,
              float(alpha), float(norm_cap), _lib.ptr(out), _lib.stream(base.device))
    return out


def n8_exact_probe_scatter_triton(output, rows, dense_probes, *, block_m=16, num_warps=4, convert_rows=True):
    """output[b, rows[b, j]] = dense_probes[b, j] in place (reference residual_repair.py:656-700)."""
    del block_m, num_warps
    if not output.is_cuda:
        raise RuntimeError("n8_exact_probe_scatter_triton requires CUDA tensors.")
    if output.ndim != 3 or rows.ndim != 2 or dense_probes.ndim != 3:
        raise RuntimeError("Expected output [BH,N,D], rows [BH,M], and dense probes [BH,M,D].")
    bh, tokens, dim = output.shape
    probes = int(rows.shape[1])
    if tuple(rows.shape) != (bh, probes) or tuple(dense_probes.shape) != (bh, probes, dim):
        raise RuntimeError(
            f"Exact-scatter shape mismatch: output={tuple(output.shape)}, "
            f"rows={tuple(rows.shape)}, probes={tuple(dense_probes.shape)}."
        )
    if rows.device != output.device or dense_probes.device != output.device:
        raise RuntimeError("Exact-scatter tensors must share a CUDA device.")
    if not dense_probes.dtype.is_floating_point:
        raise RuntimeError("Exact-scatter dense probes must be floating point.")
    if output.dtype != torch.bfloat16 or not output.is_contiguous():
        raise RuntimeError("Exact-scatter output must be a contiguous bfloat16 tensor.")
    rows_input = rows.to(torch.int32).contiguous() if convert_rows else rows.contiguous()
    dense = dense_probes.contiguous()
    if dense.dtype not in (torch.bfloat16, torch.float32):
        dense = dense.float()
    _lib.call("spr_probe_scatter", _lib.ptr(dense), _lib.DTYPE_CODE[dense.dtype], _lib.ptr(rows_input), bh, tokens,
              probes, dim, _lib.ptr(output), _lib.stream(output.device))
    return output
