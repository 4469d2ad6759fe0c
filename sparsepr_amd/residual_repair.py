"""Current-step reduced-rank residual repair (drop-in for the reference's
src/sparsepr/models/cosmos3/residual_repair.py).

Probe selection, the fit-input gathers, the reduced-rank fit (csrc/spr_rrr.hip: primal
or dual ridge solve, raw or fitted output basis, with or without weights), the
non-finite state recovery, the low-rank apply and the exact probe scatter are HIP
kernels.  Configurations outside the kernels' limits (M or D > 128, P > 128 outside the dual
form's LDS bound, rank > 64) raise instead of falling back to another implementation.
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
    """Weighted batched ridge reduced-rank regression in fp32 (reference :263-465), on
    spr_rrr_fit_ex.  Returns (x_mean [BH,1,P], x_scale [BH,1,P], y_mean [BH,1,D],
    left [BH,P,r], basis [BH,D,r]).

    M < P solves in dual form, M >= P in primal form (both fit_backend values: they
    differ in the factorisation the reference calls, not in the solution).  The basis is
    the top-r eigenvectors of the weighted output gram of the raw residual or of the
    fitted values; the "full" route and the "skinny" row-gram route with the eigh or SVD
    backends compute that subspace.  The "skinny" route with M < D and "triton_top16"
    (the reference's GPU N8 repair) takes the fixed-count subspace iteration of
    top16_right_basis_triton instead, as the reference does (:435-451, :497-503): an
    approximation that is not the exact eigenbasis.  cache_identity has no effect here."""
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
    top16 = (output_basis_backend == "skinny" and x_fit.shape[1] < y_fit.shape[2]
             and decomposition_backend == "triton_top16")
    if top16:
        if rank != 16:
            raise RuntimeError(f"triton_top16 requires rank=16, got {rank}.")
        if (int(x_fit.shape[1]), int(y_fit.shape[2])) != (64, 128):
            raise RuntimeError(
                f"N8 top-16 kernel requires [BH,64,128], got {(int(x_fit.shape[0]), int(x_fit.shape[1]), int(y_fit.shape[2]))}.")
    return _rrr_fit_hip(x_fit, y_fit, weights, int(rank), float(ridge),
                        1 if basis_source == "fitted_residual" else 0, top16)


def rrr_fit_supported(m: int, p: int, d: int, rank: int) -> bool:
    """The sizes the LDS-resident fit kernels take: x_w^T lives in 128 x 129 floats, as 128
    rows of 129 (P <= 128) or, in the dual form, 64 ceil(P / 64) rows of M | 1."""
    if m > 128 or d > 128 or rank > 64 or p > 256:
        return False
    if p <= 128:
        return True
    return m < p and 64 * ((p + 63) // 64) * (m | 1) <= 128 * 129


def _rrr_fit_hip(x, y, weights, rank, ridge, basis_source=0, top16=False):
    """The fit in 4 launches (raw residual basis) or 7 (fitted values), fp32 whatever
    the input dtype; with top16 the basis comes from the top-16 subspace iteration.
    Eigenvector signs (as eigh's) are arbitrary; left . basis^T does not depend on them."""
    dev = _lib.require_gpu(x, y, weights, what="reduced-rank residual fit")
    bh, m, p = (int(v) for v in x.shape)
    d = int(y.shape[2])
    if not rrr_fit_supported(m, p, d, rank):
        raise NotImplementedError(
            f"The MI355X reduced-rank fit handles M, D <= 128, P <= 128 (or M < P <= 256 with "
            f"64 ceil(P / 64) (M | 1) <= 16512) and rank <= 64; got M={m}, P={p}, D={d}, rank={rank}.")
    if weights is not None and tuple(weights.shape) != (bh, m):
        raise RuntimeError(f"RRR weights must have shape {(bh, m)}, got {tuple(weights.shape)}.")
    x = x.float().contiguous()
    y = y.float().contiguous()
    w = None if weights is None else weights.to(device=dev, dtype=torch.float32).contiguous()
    f32 = dict(device=dev, dtype=torch.float32)
    x_mean = torch.empty((bh, 1, p), **f32)
    x_scale = torch.empty((bh, 1, p), **f32)
    y_mean = torch.empty((bh, 1, d), **f32)
    left = torch.empty((bh, p, rank), **f32)
    basis = torch.empty((bh, d, rank), **f32)
    ws_bytes = int(_lib.query("spr_rrr_fit_workspace", bh))
    ws = _lib.workspace(ws_bytes, dev)
    _lib.call("spr_rrr_fit_top16" if top16 else "spr_rrr_fit_ex", _lib.ptr(x), _lib.ptr(y), _lib.ptr(w), bh, m, p, d,
              rank, ridge, int(basis_source),
              _lib.ptr(x_mean), _lib.ptr(x_scale), _lib.ptr(y_mean), _lib.ptr(left), _lib.ptr(basis), _lib.ptr(ws),
              ws_bytes, _lib.stream(dev))
    return x_mean, x_scale, y_mean, left, basis


def reduced_rank_output_basis(weighted_fitted, *, rank, backend):
    """Top-r right singular basis of [BH, M, D] (reference :468-506).  "eigh" and the SVD
    backends: spr_rrr_output_basis, the eigenvectors of A^T A, orthonormal, ascending;
    "triton_top16": top16_right_basis_triton (rank 16, [BH, 64, 128])."""
    if weighted_fitted.ndim != 3:
        raise RuntimeError(f"weighted_fitted must have shape [BH,M,D], got {tuple(weighted_fitted.shape)}.")
    if rank <= 0 or rank > min(weighted_fitted.shape[1:]):
        raise RuntimeError(f"Invalid rank={rank} for weighted_fitted={tuple(weighted_fitted.shape)}.")
    if backend == "triton_top16":
        if rank != 16:
            raise RuntimeError(f"triton_top16 requires rank=16, got {rank}.")
        from .kernels.rrr_eigensolver import top16_right_basis_triton

        return top16_right_basis_triton(weighted_fitted)
    if backend not in {"eigh", "svd_gesvdj", "svd_gesvd"}:
        raise RuntimeError(f"Unknown exact decomposition backend {backend!r}.")
    dev = _lib.require_gpu(weighted_fitted, what="reduced-rank output basis")
    bh, m, d = (int(v) for v in weighted_fitted.shape)
    if max(m, d) > 128 or rank > 64:
        raise NotImplementedError(f"The MI355X output basis handles M, D <= 128 and rank <= 64; got M={m}, D={d}, "
                                  f"rank={rank}.")
    a = weighted_fitted.float().contiguous()
    basis = torch.empty((bh, d, int(rank)), device=dev, dtype=torch.float32)
    ws_bytes = int(_lib.query("spr_rrr_fit_workspace", bh))
    ws = _lib.workspace(ws_bytes, dev)
    _lib.call("spr_rrr_output_basis", _lib.ptr(a), bh, m, d, int(rank), _lib.ptr(basis), _lib.ptr(ws), ws_bytes,
              _lib.stream(dev))
    return basis


def recover_nonfinite_rrr_state(state, previous):
    """Per-head containment of a non-finite fit (reference :509-587) on spr_rrr_recover:
    a head with any non-finite state value takes its previous state, or a zero
    correction when there is none.  Returns (state, recovered [BH] bool, policy)."""
    if len(state) != 5:
        raise RuntimeError(f"RRR state must contain five tensors, got {len(state)}.")
    batch_heads = int(state[0].shape[0])
    if any(int(t.shape[0]) != batch_heads for t in state):
        raise RuntimeError("RRR state tensors must share their batch-head dimension.")
    if any(not torch.is_floating_point(t) for t in state):
        raise RuntimeError("RRR state tensors must be floating point.")
    if previous is None:
        policy = "zero_repair_without_previous_state"
    else:
        if len(previous) != len(state) or any(
            old.shape != new.shape or old.device != new.device or old.dtype != new.dtype
            for old, new in zip(previous, state, strict=True)
        ):
            raise RuntimeError("Previous RRR state does not match the current fit.")
        policy = "reuse_previous_finite_repair_state"
    dev = _lib.require_gpu(*state, what="RRR state recovery")
    x_mean, x_scale, y_mean, left, basis = state
    p, d, rank = int(left.shape[1]), int(basis.shape[1]), int(left.shape[2])
    shapes = [(batch_heads, 1, p), (batch_heads, 1, p), (batch_heads, 1, d), (batch_heads, p, rank),
              (batch_heads, d, rank)]
    if [tuple(t.shape) for t in state] != shapes:
        raise RuntimeError(f"RRR state shapes {[tuple(t.shape) for t in state]} do not match {shapes}.")
    cur = [t.float().contiguous() for t in state]
    prev = [None] * 5 if previous is None else [t.float().contiguous() for t in previous]
    out = [torch.empty_like(t) for t in cur]
    recovered = torch.empty((batch_heads,), device=dev, dtype=torch.uint8)
    _lib.call("spr_rrr_recover", *[_lib.ptr(t) for t in cur], *[_lib.ptr(t) for t in prev], batch_heads, p, d, rank,
              *[_lib.ptr(t) for t in out], _lib.ptr(recovered), _lib.stream(dev))
    selected = tuple(o if o.dtype == t.dtype else o.to(t.dtype) for o, t in zip(out, state))
    return selected, recovered.bool(), policy


def apply_reduced_rank_residual(base, role, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap):
    """base + alpha * correction (optional norm cap on the base norm), in base's dtype
    (reference :600-646), on the HIP apply kernel: bf16 base, D in {64, 128}, role features
    (role [BH, N, R], R in {16, 32, 48, 64}, the last R rows of left and entries of
    x_mean / x_scale) or none, rank <= 64 (padded with zero columns, which add nothing, to 16,
    32 or 64)."""
    bh, tokens, dim = (int(v) for v in base.shape)
    rank = int(left.shape[2])
    role_dim = 0 if role is None else int(role.shape[2])
    if (base.dtype != torch.bfloat16 or dim not in (64, 128) or rank > 64 or int(left.shape[1]) != dim + role_dim
            or role_dim not in (0, 16, 32, 48, 64)):
        raise NotImplementedError(
            f"The MI355X repair apply needs a bf16 base with D in (64, 128), 0, 16, 32, 48 or 64 role features and "
            f"rank <= 64; got {base.dtype}, D={dim}, role={role_dim}, rank={rank}, left={tuple(left.shape)}.")
    from .kernels.residual_repair import repair_apply_output, repair_apply_role

    padded = 16 if rank <= 16 else (32 if rank <= 32 else 64)
    if rank < padded:
        left = torch.nn.functional.pad(left.float(), (0, padded - rank))
        basis = torch.nn.functional.pad(basis.float(), (0, padded - rank))
    if role is not None:
        return repair_apply_role(base.contiguous(), role.contiguous(), x_mean.contiguous(), x_scale.contiguous(),
                                 y_mean.contiguous(), left.contiguous(), basis.contiguous(), alpha, norm_cap)
    return repair_apply_output(base.contiguous(), x_mean.contiguous(), x_scale.contiguous(), y_mean.contiguous(),
                               left.contiguous(), basis.contiguous(), alpha, norm_cap)
