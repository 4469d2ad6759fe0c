"""N8 role metrics, their factors and the small projections, on the HIP kernels of
csrc/spr_metric.hip and csrc/spr_rrr.hip (spr_sym_top_eig)."""

from __future__ import annotations

import torch

from .. import _lib

ORTHO = {"each_cholesky_qr": 0, "each_cholesky_qr2": 1, "cholesky_qr": 2, "each_qr": 3, "final_qr": 4}
RITZ = {"rayleigh_cholesky": 0, "diagonal": 1, "previous_scale": 2, "full": 3}


def role_metric(x: torch.Tensor, *, rows: torch.Tensor | None = None, sizes: torch.Tensor | None = None,
                center: bool = False, post_scale: float = 1.0) -> torch.Tensor:
    """fp32 [BH, D, D] = post_scale / max(used, 1) * sum over the used rows (x - mean)(x - mean)^T.
    x bf16 / fp32 [BH, N, D]; rows int [count] (the same sample positions for every head);
    sizes [BH, N]: only rows with size > 0 are used (query_metric_from_key_centroids)."""
    dev = _lib.require_gpu(x, rows, sizes, what="role metric")
    if x.ndim != 3:
        raise RuntimeError(f"Expected [batch_heads, tokens, dim], got {tuple(x.shape)}.")
    bh, n, d = x.shape
    xc = x if x.dtype in (torch.bfloat16, torch.float32) else x.float()
    xc = xc.contiguous()
    r = None if rows is None else rows.to(device=dev, dtype=torch.int32).contiguous()
    sz = None if sizes is None else sizes.to(device=dev, dtype=torch.int32).reshape(bh, n).contiguous()
    out = torch.empty((bh, d, d), dtype=torch.float32, device=dev)
    _lib.call("spr_role_metric", _lib.ptr(xc), _lib.DTYPE_CODE[xc.dtype], bh, n, d, _lib.ptr(r),
              0 if r is None else int(r.numel()), _lib.ptr(sz), int(bool(center)), float(post_scale), _lib.ptr(out),
              _lib.stream(dev))
    return out


def sym_top_eig(mats: torch.Tensor, rank: int, *, symmetrize: bool = True, want_values: bool = True):
    """Top-`rank` eigenpairs of symmetric [BH, n, n] fp32 matrices, ascending (as the last
    `rank` columns of torch.linalg.eigh).  Returns (vectors [BH, n, rank], values [BH, rank])."""
    dev = _lib.require_gpu(mats, what="symmetric eigensolver")
    bh, n, n2 = mats.shape
    if n != n2:
        raise RuntimeError(f"Expected batched square matrices, got {tuple(mats.shape)}.")
    m = mats.float().contiguous()
    vecs = torch.empty((bh, n, rank), dtype=torch.float32, device=dev)
    vals = torch.empty((bh, rank), dtype=torch.float32, device=dev) if want_values else None
    _lib.call("spr_sym_top_eig", _lib.ptr(m), bh, n, int(rank), int(bool(symmetrize)), _lib.ptr(vecs),
              _lib.ptr(vals), _lib.stream(dev))
    return vecs, vals


def metric_factor(metric: torch.Tensor, rank: int) -> torch.Tensor:
    """Top-rank eigenvectors of 0.5 (M + M^T) scaled by sqrt(lambda / mean lambda) (fp32)."""
    dev = _lib.require_gpu(metric, what="metric factor")
    bh, n, _ = metric.shape
    m = metric.float().contiguous()
    factor = torch.empty((bh, n, rank), dtype=torch.float32, device=dev)
    nbytes = int(_lib.query("spr_metric_factor_workspace", bh, int(rank)))
    ws = _lib.workspace(nbytes, dev)
    _lib.call("spr_metric_factor", _lib.ptr(m), bh, n, int(rank), _lib.ptr(factor), _lib.ptr(ws), ws.numel(),
              _lib.stream(dev))
    return factor


def warm_metric_factor(metric: torch.Tensor, prev_state: torch.Tensor, rank: int, *,
                       prev_factor: torch.Tensor | None = None, power_iters: int = 1,
                       orthogonalization: str = "each_cholesky_qr2", ritz_mode: str = "rayleigh_cholesky",
                       rayleigh_ridge: float = 1e-4, cholesky_qr_ridge: float = 1e-5):
    """One warm subspace update.  Returns (factor, state, recovered bool [BH]); with
    prev_factor, recovered heads keep prev_factor / prev_state.  The full finish's columns
    are in ascending eigenvalue order with the eigensolver's signs."""
    dev = _lib.require_gpu(metric, prev_state, prev_factor, what="warm metric factor")
    bh, n, _ = metric.shape
    m = metric.float().contiguous()
    ps = prev_state.float().contiguous()
    pf = None if prev_factor is None else prev_factor.float().contiguous()
    factor = torch.empty((bh, n, rank), dtype=torch.float32, device=dev)
    state = torch.empty((bh, n, rank), dtype=torch.float32, device=dev)
    rec = torch.empty((bh,), dtype=torch.uint8, device=dev)
    nbytes = int(_lib.query("spr_warm_metric_factor_workspace", bh, n, int(rank), RITZ[ritz_mode]))
    ws = _lib.workspace(nbytes, dev) if nbytes > 0 else None
    _lib.call("spr_warm_metric_factor_ex", _lib.ptr(m), _lib.ptr(ps), _lib.ptr(pf), bh, n, int(rank),
              int(power_iters), ORTHO[orthogonalization], RITZ[ritz_mode], float(rayleigh_ridge),
              float(cholesky_qr_ridge), _lib.ptr(factor), _lib.ptr(state), _lib.ptr(rec), _lib.ptr(ws), nbytes,
              _lib.stream(dev))
    return factor, state, rec.bool()


def project_rows(x: torch.Tensor, factor: torch.Tensor, *, divisor: torch.Tensor | None = None, tf32: bool = False,
                 row_rms: bool = False, eps: float = 1e-6, precision: str | None = None, weight: float = 1.0,
                 out: torch.Tensor | None = None, out_col: int = 0) -> torch.Tensor:
    """(x [BH, M, D] . factor [BH, D, r]) / divisor[h] times weight, optionally row-RMS
    normalised; fp32 [BH, M, r], or columns out_col .. out_col + r of out [BH, M, C].  The
    operands are fp32, or both rounded to TF32 (tf32, or precision "high") or to bf16
    (precision "medium"); precision "highest" is fp32."""
    dev = _lib.require_gpu(x, factor, divisor, out, what="row projection")
    if x.ndim != 3 or factor.ndim != 3 or x.shape[0] != factor.shape[0] or x.shape[2] != factor.shape[1]:
        raise RuntimeError(f"Projection shape mismatch: x={tuple(x.shape)}, factor={tuple(factor.shape)}.")
    bh, m, d = x.shape
    r = factor.shape[2]
    prec = 1 if tf32 else 0
    if precision is not None:
        prec = {"highest": 0, "high": 1, "medium": 2}[precision]
    xc = x.float().contiguous()
    fc = factor.float().contiguous()
    dv = None if divisor is None else divisor.float().reshape(bh).contiguous()
    if out is None:
        out = torch.empty((bh, m, r), dtype=torch.float32, device=dev)
    elif (out.ndim != 3 or tuple(out.shape[:2]) != (bh, m) or out.dtype != torch.float32 or not out.is_contiguous()
          or out_col < 0 or out_col + r > out.shape[2]):
        raise RuntimeError(f"Projection output must be contiguous fp32 [{bh}, {m}, >= {out_col + r}].")
    _lib.call("spr_project_rows_ex", _lib.ptr(xc), _lib.ptr(fc), _lib.ptr(dv), bh, m, d, r, prec, int(bool(row_rms)),
              float(eps), float(weight), _lib.ptr(out), int(out.shape[2]), int(out_col), _lib.stream(dev))
    return out


def original_centroids(x: torch.Tensor, y: torch.Tensor | None, sorted_idx: torch.Tensor, offsets: torch.Tensor,
                       n_clusters: int, x_fallback: torch.Tensor | None = None,
                       y_fallback: torch.Tensor | None = None):
    """fp32 cluster means of x (and y, in the same traversal); empty clusters take the
    fallback rows (zeros without one).  Returns x_means (, y_means)."""
    dev = _lib.require_gpu(x, y, sorted_idx, offsets, what="original centroids")
    bh, n, d = x.shape
    if y is not None and (y.shape != x.shape or y.dtype != x.dtype):
        raise RuntimeError(f"Joint centroids need matching x/y, got {tuple(x.shape)} {x.dtype} / "
                           f"{tuple(y.shape)} {y.dtype}.")
    xc = x if x.dtype in (torch.bfloat16, torch.float32) else x.float()
    yc = None if y is None else (y if y.dtype == xc.dtype else y.to(xc.dtype))
    xc = xc.contiguous()
    yc = None if yc is None else yc.contiguous()
    shape = (bh, int(n_clusters), d)

    def fb(t):
        if t is None:
            return None
        if tuple(t.shape) != shape:
            raise RuntimeError(f"Empty-centroid fallback mismatch: fallback={tuple(t.shape)}, means={shape}.")
        return t.to(device=dev, dtype=torch.float32).contiguous()

    xf, yf = fb(x_fallback), fb(y_fallback)
    x_out = torch.empty(shape, dtype=torch.float32, device=dev)
    y_out = None if yc is None else torch.empty(shape, dtype=torch.float32, device=dev)
    nbytes = int(_lib.query("spr_original_centroids_workspace", bh, n, int(n_clusters), d))
    ws = _lib.workspace(nbytes, dev) if nbytes > 0 else None
    _lib.call("spr_original_centroids", _lib.ptr(xc), _lib.ptr(yc), _lib.DTYPE_CODE[xc.dtype],
              _lib.ptr(sorted_idx.to(torch.int32).contiguous()), _lib.ptr(offsets.to(torch.int32).contiguous()),
              bh, n, int(n_clusters), d, _lib.ptr(xf), _lib.ptr(yf), _lib.ptr(x_out), _lib.ptr(y_out), _lib.ptr(ws),
              nbytes, _lib.stream(dev))
    return x_out if y_out is None else (x_out, y_out)
