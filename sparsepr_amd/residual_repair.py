"""Current-step reduced-rank residual repair (drop-in for the reference's
src/sparsepr/models/cosmos3/residual_repair.py).

Probe selection, the fit-input gathers, the low-rank apply and the exact probe
scatter are HIP kernels.  The fit itself is small batched linear algebra
([BH, M, P] with M, P <= 128) and runs on the GPU through torch.linalg in fp32,
with the reference's branch structure (dual Cholesky for M < P, primal solve
otherwise; eigen basis of the weighted residual).
"""

from __future__ import annotations

import torch

from . import _lib

_IDENTITY_CACHE: dict = {}

MODE_VECTORIZED = 0
MODE_ROUNDS = 1
MODE_FIRST_TOKEN = 2


def cached_identity(size: int, *, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    key = (torch.device(device).type, torch.device(device).index, dtype, int(size))
    value = _IDENTITY_CACHE.get(key)
    if value is None:
        value = torch.eye(size, device=device, dtype=dtype)
        _IDENTITY_CACHE[key] = value
    return value


def _check_probe_inputs(role_features, role_labels):
    if role_features.ndim != 3 or role_labels.shape != role_features.shape[:2]:
        raise RuntimeError(
            "Role probe selection expects features [BH,N,R] and labels [BH,N], got "
            f"features={tuple(role_features.shape)}, labels={tuple(role_labels.shape)}."
        )
    return _lib.require_gpu(role_features, role_labels, what="probe selection")


def group_centers(features: torch.Tensor, labels: torch.Tensor, num_clusters: int):
    """fp32 cluster centers (fp64 sums / size) and sizes int32 [BH, C]."""
    from .flash_kmeans.kmeans_impl import centroid_update_sorted
    from .kernels.permute import argsort_labels

    bh, n, r = features.shape
    lab = labels.to(torch.int32).contiguous()
    idx, sizes, offsets = argsort_labels(lab, num_clusters)
    x = features if features.dtype in (torch.bfloat16, torch.float32) else features.float()
    old = torch.zeros((bh, num_clusters, r), dtype=x.dtype, device=x.device)
    res = centroid_update_sorted(x, lab, old, want_mean32=True, sorted_idx=idx, sizes=sizes, offsets=offsets)
    return res.mean32, sizes


def select_probes(features: torch.Tensor, labels: torch.Tensor, num_clusters: int, rows: int, mode: int,
                  centers: torch.Tensor | None = None, sizes: torch.Tensor | None = None):
    """HIP probe selection.  Returns (rows int64 [BH, M], weights fp32 [BH, M]).
    `centers` (fp32 [BH, C, R]) and `sizes` (int32 [BH, C]) may be passed when
    the caller already has them (the k-means of the same labels)."""
    dev = _check_probe_inputs(features, labels)
    bh, n, r = features.shape
    count = min(max(1, int(rows)), int(n))
    lab = labels.to(torch.int32).contiguous()
    f = features if features.dtype in (torch.bfloat16, torch.float32) else features.float()
    f = f.contiguous()
    dist = None
    if mode != MODE_FIRST_TOKEN:
        if centers is None or sizes is None:
            centers, sizes = group_centers(f, lab, num_clusters)
        dist = torch.empty((bh, n), dtype=torch.float32, device=dev)
        _lib.call("spr_probe_distances", _lib.ptr(f), _lib.DTYPE_CODE[f.dtype], _lib.ptr(lab),
                  _lib.ptr(centers.float().contiguous()), bh, n, num_clusters, r, _lib.ptr(dist), _lib.stream(dev))
    elif sizes is None:
        from .kernels.permute import argsort_labels

        sizes = argsort_labels(lab, num_clusters)[1]
    out_rows = torch.empty((bh, count), dtype=torch.int32, device=dev)
    weights = torch.empty((bh, count), dtype=torch.float32, device=dev)
    ws_bytes = int(_lib.query("spr_probe_select_workspace", bh, num_clusters))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    _lib.call("spr_probe_select", _lib.ptr(dist), _lib.ptr(lab), _lib.ptr(sizes.to(torch.int32).contiguous()), bh,
              n, num_clusters, count, mode, _lib.ptr(out_rows), _lib.ptr(weights), None, _lib.ptr(ws), ws_bytes,
              _lib.stream(dev))
    return out_rows.long(), weights


def select_role_equal_probes(role_features, role_labels, *, num_clusters, rows):
    """Representative-first equal-coverage probes per head (reference :36-115);
    works for rows > num_clusters (several representative rounds)."""
    return select_probes(role_features, role_labels, num_clusters, rows, MODE_ROUNDS)


def select_role_equal_probes_vectorized(role_features, role_labels, *, num_clusters, rows):
    """One representative per group for rows <= num_clusters (reference :118-208)."""
    _check_probe_inputs(role_features, role_labels)
    count = min(max(1, int(rows)), int(role_features.shape[1]))
    if count > int(num_clusters):
        raise RuntimeError(
            "Vectorized role probes currently require rows <= num_clusters; "
            f"got rows={count}, clusters={num_clusters}."
        )
    return select_probes(role_features, role_labels, num_clusters, rows, MODE_VECTORIZED)


def select_first_token_largest_groups(role_features, role_labels, *, num_clusters, rows):
    """First token of each of the largest groups, weight ~ group size (reference :211-260)."""
    _check_probe_inputs(role_features, role_labels)
    count = min(max(1, int(rows)), int(role_features.shape[1]))
    if count > int(num_clusters):
        raise RuntimeError(
            "First-token role probes require rows <= num_clusters; "
            f"got rows={count}, clusters={num_clusters}."
        )
    return select_probes(role_features, role_labels, num_clusters, rows, MODE_FIRST_TOKEN)


def fit_reduced_rank_residual(x_fit, y_fit, *, rank, ridge, weights=None, output_basis_backend="full",
                              cache_identity=False, fit_backend="standard", decomposition_backend="eigh",
                              basis_source="fitted_residual"):
    """Weighted batched ridge reduced-rank regression in fp32 (reference :263-465).

    Returns (x_mean [BH,1,P], x_scale [BH,1,P], y_mean [BH,1,D], left [BH,P,r], basis [BH,D,r]).
    decomposition_backend "triton_top16" (the reference's approximate top-16 power
    iteration) is served by the exact eigen decomposition."""
    with torch.autocast(device_type=x_fit.device.type, enabled=False):
        return _fit_fp32(x_fit, y_fit, rank=rank, ridge=ridge, weights=weights,
                         output_basis_backend=output_basis_backend, cache_identity=cache_identity,
                         fit_backend=fit_backend, decomposition_backend=decomposition_backend,
                         basis_source=basis_source)


def _fit_fp32(x_fit, y_fit, *, rank, ridge, weights, output_basis_backend, cache_identity, fit_backend,
              decomposition_backend, basis_source):
    if x_fit.ndim != 3 or y_fit.ndim != 3 or x_fit.shape[:2] != y_fit.shape[:2]:
        raise RuntimeError(
            "RRR expects X=[BH,M,P] and Y=[BH,M,D] with matching BH/M, got "
            f"X={x_fit.shape}, Y={y_fit.shape}."
        )
    if rank <= 0 or rank > y_fit.shape[2] or rank > x_fit.shape[1]:
        raise RuntimeError(f"Invalid RRR rank={rank} for X={tuple(x_fit.shape)}, Y={tuple(y_fit.shape)}.")
    if ridge < 0.0:
        raise RuntimeError(f"RRR ridge must be non-negative, got {ridge}.")
    if output_basis_backend not in {"full", "skinny"}:
        raise RuntimeError(f"RRR output_basis_backend must be 'full' or 'skinny', got {output_basis_backend!r}.")
    if fit_backend not in {"standard", "dual_cholesky"}:
        raise RuntimeError(f"RRR fit_backend must be 'standard' or 'dual_cholesky', got {fit_backend!r}.")
    if decomposition_backend not in {"eigh", "svd_gesvdj", "svd_gesvd", "triton_top16"}:
        raise RuntimeError(
            "RRR decomposition_backend must be 'eigh', 'svd_gesvdj', "
            f"'svd_gesvd', or 'triton_top16'; got {decomposition_backend!r}."
        )
    if basis_source not in {"fitted_residual", "raw_residual"}:
        raise RuntimeError(f"RRR basis_source must be 'fitted_residual' or 'raw_residual', got {basis_source!r}.")
    x = x_fit.float()
    y = y_fit.float()
    if _rrr_fit_fused(x, y, weights, rank, output_basis_backend, basis_source):
        return _rrr_fit_hip(x, y, weights, int(rank), float(ridge))
    if weights is None:
        w = torch.ones((*x.shape[:2], 1), device=x.device, dtype=torch.float32)
        x_mean = x.mean(dim=1, keepdim=True)
        x_scale = x.std(dim=1, keepdim=True).clamp_min(1e-5)
        y_mean = y.mean(dim=1, keepdim=True)
    else:
        if weights.shape != x.shape[:2]:
            raise RuntimeError(f"RRR weights must have shape {tuple(x.shape[:2])}, got {tuple(weights.shape)}.")
        w = weights.to(device=x.device, dtype=torch.float32).unsqueeze(2)
        w_sum = w.sum(dim=1, keepdim=True).clamp_min(1e-20)
        x_mean = (w * x).sum(dim=1, keepdim=True) / w_sum
        x_var = (w * (x - x_mean).square()).sum(dim=1, keepdim=True) / w_sum
        x_scale = x_var.sqrt().clamp_min(1e-5)
        y_mean = (w * y).sum(dim=1, keepdim=True) / w_sum
    xn = (x - x_mean) / x_scale
    yc = y - y_mean
    sw = w.sqrt()
    xw = xn * sw
    yw = yc * sw
    p = int(x.shape[2])
    m = int(x.shape[1])
    dual = None
    weight = None
    fitted = None
    weighted_fitted = None

    def eye(size):
        base = cached_identity(size, device=x.device, dtype=torch.float32) if cache_identity else \
            torch.eye(size, device=x.device, dtype=torch.float32)
        return base.expand(x.shape[0], -1, -1)

    if m < p:
        gram = torch.bmm(xw, xw.transpose(1, 2))
        if fit_backend == "dual_cholesky":
            gram.diagonal(dim1=1, dim2=2).add_(float(ridge))
            factor, _info = torch.linalg.cholesky_ex(gram, check_errors=False)
            dual = torch.cholesky_solve(yw, factor)
            weighted_fitted = torch.add(yw, dual, alpha=-float(ridge))
        else:
            dual = torch.linalg.solve_ex(gram + float(ridge) * eye(m), yw)[0]
            weight = torch.bmm(xw.transpose(1, 2), dual)
            fitted = torch.bmm(xn, weight)
    else:
        gram = torch.bmm(xw.transpose(1, 2), xw)
        rhs = torch.bmm(xw.transpose(1, 2), yw)
        weight = torch.linalg.solve_ex(gram + float(ridge) * eye(p), rhs)[0]
        fitted = torch.bmm(xn, weight)
    if output_basis_backend == "skinny" and m < int(y.shape[2]):
        if basis_source == "raw_residual":
            basis_input = yw
        else:
            if weighted_fitted is None:
                weighted_fitted = fitted * sw
            basis_input = weighted_fitted
        basis = reduced_rank_output_basis(basis_input, rank=int(rank), backend=decomposition_backend)
    else:
        values = yc if basis_source == "raw_residual" else fitted
        if values is None:  # dual Cholesky with the full basis: materialise the fit
            values = torch.bmm(xn, torch.bmm(xw.transpose(1, 2), dual))
        output_gram = torch.bmm(values.transpose(1, 2), values * w)
        _evals, evecs = torch.linalg.eigh(output_gram)
        basis = evecs[:, :, -int(rank):].contiguous()
    if dual is not None and weight is None:
        left = torch.bmm(xw.transpose(1, 2), torch.bmm(dual, basis)).contiguous()
    else:
        left = torch.bmm(weight, basis).contiguous()
    return x_mean, x_scale, y_mean, left, basis


def _rrr_fit_fused(x, y, weights, rank, output_basis_backend, basis_source):
    """Whether the fit is the one spr_rrr_fit computes in one kernel: weights given,
    M >= P (primal ridge solve), the eigen basis of the raw weighted residual, every
    dimension at most 128 and rank at most 16, on the GPU."""
    bh, m, p = (int(v) for v in x.shape)
    d = int(y.shape[2])
    if not (x.is_cuda and weights is not None and basis_source == "raw_residual"):
        return False
    if output_basis_backend == "skinny" and m < d:
        return False
    return bh > 0 and p <= m <= 128 and d <= 128 and int(rank) <= 16


def _rrr_fit_hip(x, y, weights, rank, ridge):
    """Weighted standardisation, primal ridge solve and the top-rank eigenvectors of
    y_w^T y_w in four launches (reference :364-384, :424-434, :449-456, :463-464).
    Eigenvector signs (as eigh's) are arbitrary; left . basis^T does not depend on them."""
    dev = _lib.require_gpu(x, y, weights, what="reduced-rank residual fit")
    if weights.shape != x.shape[:2]:
        raise RuntimeError(f"RRR weights must have shape {tuple(x.shape[:2])}, got {tuple(weights.shape)}.")
    bh, m, p = (int(v) for v in x.shape)
    d = int(y.shape[2])
    x = x.contiguous()
    y = y.contiguous()
    w = weights.to(device=dev, dtype=torch.float32).contiguous()
    f32 = dict(device=dev, dtype=torch.float32)
    x_mean = torch.empty((bh, 1, p), **f32)
    x_scale = torch.empty((bh, 1, p), **f32)
    y_mean = torch.empty((bh, 1, d), **f32)
    left = torch.empty((bh, p, rank), **f32)
    basis = torch.empty((bh, d, rank), **f32)
    ws_bytes = int(_lib.query("spr_rrr_fit_workspace", bh))
    ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
    _lib.call("spr_rrr_fit", _lib.ptr(x), _lib.ptr(y), _lib.ptr(w), bh, m, p, d, rank, ridge, _lib.ptr(x_mean),
              _lib.ptr(x_scale), _lib.ptr(y_mean), _lib.ptr(left), _lib.ptr(basis), _lib.ptr(ws), ws_bytes,
              _lib.stream(dev))
    return x_mean, x_scale, y_mean, left, basis


def reduced_rank_output_basis(weighted_fitted, *, rank, backend):
    """Top-r right singular basis of [BH, M, D] via the M x M row gram (reference :468-506)."""
    if weighted_fitted.ndim != 3:
        raise RuntimeError(f"weighted_fitted must have shape [BH,M,D], got {tuple(weighted_fitted.shape)}.")
    if rank <= 0 or rank > min(weighted_fitted.shape[1:]):
        raise RuntimeError(f"Invalid rank={rank} for weighted_fitted={tuple(weighted_fitted.shape)}.")
    if backend in {"eigh", "triton_top16"}:
        row_gram = torch.bmm(weighted_fitted, weighted_fitted.transpose(1, 2))
        eigenvalues, left_vectors = torch.linalg.eigh(row_gram)
        left_vectors = left_vectors[:, :, -rank:]
        scales = eigenvalues[:, -rank:].clamp_min(1e-20).rsqrt().unsqueeze(1)
        return (torch.bmm(weighted_fitted.transpose(1, 2), left_vectors) * scales).contiguous()
    if backend not in {"svd_gesvdj", "svd_gesvd"}:
        raise RuntimeError(f"Unknown exact decomposition backend {backend!r}.")
    _u, _s, vh = torch.linalg.svd(weighted_fitted, full_matrices=False)
    return vh[:, :rank, :].transpose(1, 2).contiguous()


def recover_nonfinite_rrr_state(state, previous):
    """Per-head containment of a non-finite fit (reference :509-587): reuse the
    head's previous state, or a zero correction when there is none."""
    if len(state) != 5:
        raise RuntimeError(f"RRR state must contain five tensors, got {len(state)}.")
    batch_heads = int(state[0].shape[0])
    if any(int(t.shape[0]) != batch_heads for t in state):
        raise RuntimeError("RRR state tensors must share their batch-head dimension.")
    recovered = torch.zeros(batch_heads, device=state[0].device, dtype=torch.bool)
    for t in state:
        if not torch.is_floating_point(t):
            raise RuntimeError("RRR state tensors must be floating point.")
        recovered |= ~torch.isfinite(t).reshape(batch_heads, -1).all(dim=1)
    if previous is None:
        fallback = (torch.zeros_like(state[0]), torch.ones_like(state[1]), torch.zeros_like(state[2]),
                    torch.zeros_like(state[3]), torch.zeros_like(state[4]))
        policy = "zero_repair_without_previous_state"
    else:
        if len(previous) != len(state) or any(
            old.shape != new.shape or old.device != new.device or old.dtype != new.dtype
            for old, new in zip(previous, state, strict=True)
        ):
            raise RuntimeError("Previous RRR state does not match the current fit.")
        fallback = previous
        policy = "reuse_previous_finite_repair_state"
    selected = tuple(
        torch.where(recovered.reshape(batch_heads, *((1,) * (cur.ndim - 1))), old, cur)
        for cur, old in zip(state, fallback, strict=True)
    )
    return selected, recovered, policy


def apply_reduced_rank_residual(base, role, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap):
    """base + alpha * correction (optional norm cap), cast to base.dtype (reference :620-646).
    Output-only bf16 rank-16 states with D in {64, 128} use the HIP apply kernel;
    other shapes (role features, other ranks) use torch ops on the GPU."""
    if (role is None and base.is_cuda and base.dtype == torch.bfloat16 and base.shape[2] in (64, 128)
            and left.shape[2] == 16 and left.shape[1] == base.shape[2]):
        from .kernels.residual_repair import repair_apply_output

        return repair_apply_output(base.contiguous(), x_mean.contiguous(), x_scale.contiguous(),
                                   y_mean.contiguous(), left.contiguous(), basis.contiguous(), alpha, norm_cap)
    base_dim = int(base.shape[2])
    coords = torch.bmm((base.float() - x_mean[:, :, :base_dim]) / x_scale[:, :, :base_dim], left[:, :base_dim])
    if role is not None:
        coords = coords + torch.bmm((role.float() - x_mean[:, :, base_dim:]) / x_scale[:, :, base_dim:],
                                    left[:, base_dim:])
    correction = torch.bmm(coords, basis.transpose(1, 2)) + y_mean
    if norm_cap > 0.0:
        cn = torch.linalg.vector_norm(correction, dim=2, keepdim=True).clamp_min(1e-20)
        bn = torch.linalg.vector_norm(base.float(), dim=2, keepdim=True)
        correction = correction * (float(norm_cap) * bn / cn).clamp_max(1.0)
    return (base.float() + float(alpha) * correction).to(base.dtype)
