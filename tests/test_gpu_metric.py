"""GPU parity of the N8 role-metric kernels: metric covariances, the top-r symmetric
eigensolver, the cold metric factor, the warm subspace update (with its recovery), the
centroid projections and the original-space (joint) centroids, each against the float64
oracle.  Tolerances are fp32 accumulation tolerances, stated per test."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _spectrum(rng, bh, d, eig):
    qm = np.linalg.qr(rng.standard_normal((bh, d, d)))[0]
    return np.einsum("bij,j,bkj->bik", qm, eig, qm).astype(np.float32), qm


def test_role_metric_sampled_and_masked(dev, oracle):
    """key_metric_from_queries (bf16 rows at the deterministic sample, uncentred) and
    query_metric_from_key_centroids (fp32 centroids, empty clusters left out, centred, / D):
    relative Frobenius error <= 1e-5 against float64."""
    from sparsepr_amd import operator_kmeans as ok

    rng = np.random.default_rng(61)
    q = oracle.to_bf16((rng.standard_normal((2, 5000, 128)) + 0.3).astype(np.float32))
    got = ok.key_metric_from_queries(to_dev(q, dev, torch.bfloat16), 2048)
    pos = ok.deterministic_token_positions(5000, 2048, dev).cpu().numpy()
    assert pos.size == 2048 and pos[0] == 0 and pos[-1] == 4999 and (np.diff(pos) > 0).all()
    assert _rel(got.cpu().numpy(), oracle.role_metric(q, rows=pos)) <= 1e-5
    cent = rng.standard_normal((3, 300, 128)).astype(np.float32)
    sizes = rng.integers(0, 50, (3, 300))
    sizes[:, ::9] = 0
    got = ok.query_metric_from_key_centroids(to_dev(cent, dev), to_dev(sizes, dev))
    ref = oracle.role_metric(cent, sizes=sizes, center=True, post_scale=1.0 / 128)
    assert _rel(got.cpu().numpy(), ref) <= 1e-5
    # centred covariance of all rows, bf16 input (value_metric_from_values with a full sample)
    v = oracle.to_bf16(rng.standard_normal((1, 1500, 64)).astype(np.float32))
    got = ok.value_metric_from_values(to_dev(v, dev, torch.bfloat16), 4096)
    assert _rel(got.cpu().numpy(), oracle.role_metric(v, center=True)) <= 1e-5


@pytest.mark.parametrize("n,rank", [(128, 16), (128, 48), (128, 64), (64, 64), (100, 33), (128, 5), (48, 48),
                                    (16, 16)])
def test_sym_top_eig_matches_eigh(dev, oracle, n, rank):
    """Eigenvalues (Rayleigh quotients) within 1e-5 of the spectral norm of numpy's; the basis
    orthonormal to 1e-5; the projector on the top-`rank` subspace equal to numpy's to 1e-4
    (the spectrum has a gap at `rank`, distinct values below it and a cluster of three
    equal eigenvalues above it)."""
    from sparsepr_amd.kernels.role_metric import sym_top_eig

    rng = np.random.default_rng(n + rank)
    eig = np.sort(rng.uniform(0.0, 1.0, n))
    eig[-rank:] = np.sort(rng.uniform(2.0, 10.0, rank))
    if rank >= 6:
        eig[-4:-1] = eig[-4]  # a cluster of three
        eig = np.sort(eig)
    m, _ = _spectrum(rng, 3, n, eig)
    vecs, vals = sym_top_eig(to_dev(m, dev), rank)
    v = vecs.cpu().numpy().astype(np.float64)
    w, u = np.linalg.eigh(m.astype(np.float64))
    assert np.abs(vals.cpu().numpy() - w[:, -rank:]).max() <= 1e-5 * np.abs(w).max()
    assert np.abs(np.einsum("bir,bis->brs", v, v) - np.eye(rank)).max() <= 1e-5
    p_gpu = np.einsum("bir,bjr->bij", v, v)
    p_ref = np.einsum("bir,bjr->bij", u[:, :, -rank:], u[:, :, -rank:])
    assert np.abs(p_gpu - p_ref).max() <= 1e-4
    # distinct eigenvalues: each vector matches numpy's up to sign
    dots = np.abs(np.einsum("bir,bir->br", v, u[:, :, -rank:]))
    distinct = np.ones(rank, bool)
    for c in range(rank):
        lam = w[0, n - rank + c]
        distinct[c] = (np.abs(w[0] - lam) > 1e-3 * np.abs(w[0]).max()).sum() == n - 1
    assert (dots[:, distinct] > 1 - 1e-4).all()


def test_metric_factor_cold(dev, oracle):
    """F F^T of the cold factor of a K metric (the sampled Q second moment) against the
    float64 metric_factor: relative Frobenius error <= 1e-3 (a continuous spectrum: the eigengap
    at the cut sets how far fp32 rounding turns the subspace)."""
    from sparsepr_amd import operator_kmeans as ok

    rng = np.random.default_rng(62)
    basis = rng.standard_normal((2, 128, 128)).astype(np.float32) * np.linspace(0.05, 2.0, 128)[None, None]
    q = oracle.to_bf16(np.einsum("bnd,bed->bne", rng.standard_normal((2, 4000, 128)).astype(np.float32), basis))
    metric = ok.key_metric_from_queries(to_dev(q, dev, torch.bfloat16), 2048)
    for rank in (48, 64):
        f = ok.metric_factor(metric, rank).cpu().numpy().astype(np.float64)
        ref = oracle.metric_factor(metric.cpu().numpy(), rank)
        assert _rel(np.einsum("bir,bjr->bij", f, f), np.einsum("bir,bjr->bij", ref, ref)) <= 1e-3
    bad = metric.clone()
    bad[1, 3, 3] = float("nan")
    with pytest.raises(RuntimeError, match="non-finite"):
        ok.metric_factor(bad, 48)


@pytest.mark.parametrize("ortho,ritz", [("each_cholesky_qr2", "rayleigh_cholesky"),
                                        ("each_cholesky_qr", "diagonal"),
                                        ("cholesky_qr", "previous_scale"),
                                        ("each_qr", "full"),
                                        ("each_qr", "rayleigh_cholesky"),
                                        ("final_qr", "diagonal"),
                                        ("final_qr", "full"),
                                        ("each_cholesky_qr2", "full")])
def test_warm_subspace_factor(dev, oracle, ortho, ritz):
    """The warm update against the float64 restatement from the same previous basis: factor
    within 2e-3 of its largest entry, basis within 1e-3 (the Householder bases carry LAPACK's
    signs, so they compare entry by entry too); the full finish's columns have the
    eigensolver's signs, so its factor is compared through F F^T (1e-4 relative) and its
    column norms (ascending eigenvalues).  A NaN metric head is reported recovered and, with
    prev_factor, keeps the previous factor and state."""
    from sparsepr_amd import operator_kmeans as ok
    from sparsepr_amd.kernels.role_metric import warm_metric_factor

    rng = np.random.default_rng(63)
    d, r = 128, 64
    eig = np.concatenate([np.linspace(0.01, 0.5, d - r), np.linspace(1.0, 20.0, r)])
    m, qm = _spectrum(rng, 3, d, eig)
    prev = (qm[:, :, -r:] + 0.05 * rng.standard_normal((3, d, r))).astype(np.float32)
    f, b, rec = ok.warm_subspace_metric_factor(to_dev(m, dev), to_dev(prev, dev), r, power_iters=2,
                                               orthogonalization=ortho, ritz_mode=ritz, rayleigh_ridge=1e-4,
                                               cholesky_qr_ridge=1e-5, return_basis=True, return_recovery_mask=True)
    rf, rb, rrec = oracle.warm_subspace_metric_factor(m, prev, r, 2, ortho, ritz, 1e-4, 1e-5)
    assert not rec.any() and not rrec.any()
    fn, bn = f.cpu().numpy(), b.cpu().numpy()
    if ritz == "full":
        assert _rel(np.einsum("bir,bjr->bij", fn, fn), np.einsum("bir,bjr->bij", rf, rf)) <= 1e-4
        assert np.abs(np.linalg.norm(fn, axis=1) - np.linalg.norm(rf, axis=1)).max() <= 1e-4 * np.abs(rf).max()
    else:
        assert np.abs(fn - rf).max() <= 2e-3 * np.abs(rf).max()
    assert np.abs(bn - rb).max() <= 1e-3
    bad = m.copy()
    bad[2, 0, 5] = np.nan
    prev_f = rng.standard_normal((3, d, r)).astype(np.float32)
    f2, s2, rec2 = warm_metric_factor(to_dev(bad, dev), to_dev(prev, dev), r, prev_factor=to_dev(prev_f, dev),
                                      power_iters=2, orthogonalization=ortho, ritz_mode=ritz)
    assert rec2.cpu().tolist() == [False, False, True]
    assert np.array_equal(f2[2].cpu().numpy(), prev_f[2]) and np.array_equal(s2[2].cpu().numpy(), prev[2])
    f2n = f2[:2].cpu().numpy()
    if ritz == "full":
        assert _rel(np.einsum("bir,bjr->bij", f2n, f2n), np.einsum("bir,bjr->bij", rf[:2], rf[:2])) <= 1e-4
    else:
        assert np.abs(f2n - rf[:2]).max() <= 2e-3 * np.abs(rf).max()


def test_project_rows(dev, oracle):
    """The compiled K-centroid projection (TF32 operands, / key scale) and the Q-centroid
    projection (fp32, row RMS with eps 1e-6): relative error <= 1e-6 per element scale."""
    from sparsepr_amd.kernels.role_metric import project_rows

    rng = np.random.default_rng(64)
    x = rng.standard_normal((2, 1000, 128)).astype(np.float32)
    f = rng.standard_normal((2, 128, 48)).astype(np.float32) / 10
    div = np.array([1.7, 0.3], np.float32)
    got = project_rows(to_dev(x, dev), to_dev(f, dev), divisor=to_dev(div, dev), tf32=True).cpu().numpy()
    ref = oracle.project_rows(x, f, div=div, tf32=True)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max() * 8
    got = project_rows(to_dev(x, dev), to_dev(f[:, :, :40], dev), row_rms=True).cpu().numpy()
    ref = oracle.project_rows(x, f[:, :, :40], row_rms=True)
    assert np.abs(got - ref).max() <= 1e-5


@pytest.mark.parametrize("k,joint", [(300, True), (4, True), (100, False), (50, True)])  # k = 4: split clusters
def test_original_centroids_exact(dev, oracle, k, joint):
    """fp32 means of bf16 K (and V) under labels, empty clusters from the fp32 fallback or
    zeros: bit-exact against the float64 sums (exact for bf16 rows) rounded to fp32."""
    from sparsepr_amd import operator_kmeans as ok
    from sparsepr_amd.kernels.centroid_reduction import joint_original_centroids_triton, original_centroids_triton

    rng = np.random.default_rng(65 + k)
    n, d = 5000, 128
    x = oracle.to_bf16(rng.standard_normal((2, n, d)).astype(np.float32))
    y = oracle.to_bf16(rng.standard_normal((2, n, d)).astype(np.float32))
    labels = rng.integers(0, k, (2, n)).astype(np.int32)
    if k == 50:
        labels[rng.random((2, n)) < 0.7] = 2  # one cluster of several 512-row slices, the rest one each
    labels[labels == 1] = 0  # cluster 1 empty
    sizes = np.stack([np.bincount(r, minlength=k) for r in labels])
    fb = rng.standard_normal((2, k, d)).astype(np.float32)
    _, rx, _ = oracle.centroid_update(x, labels, fb, out_bf16=False)
    _, ry, _ = oracle.centroid_update(y, labels, np.zeros_like(fb), out_bf16=False)
    xt, yt = to_dev(x, dev, torch.bfloat16), to_dev(y, dev, torch.bfloat16)
    lt, st = to_dev(labels, dev), to_dev(sizes, dev)
    if joint:
        gx, gy = ok.joint_original_centroids(xt, yt, lt, st, x_empty_fallback=to_dev(fb, dev))
        assert np.array_equal(gy.cpu().numpy(), ry)
        tx, ty = joint_original_centroids_triton(xt, yt, lt, st, x_empty_fallback=to_dev(fb, dev))
        assert torch.equal(tx, gx) and torch.equal(ty, gy)
    else:
        gx = ok.original_centroids(xt, lt, st, empty_fallback=to_dev(fb, dev))
        assert torch.equal(original_centroids_triton(xt, lt, st, empty_fallback=to_dev(fb, dev)), gx)
        gz = ok.original_centroids(xt, lt, st)
        assert (gz[:, 1].cpu().numpy() == 0).all()
    assert np.array_equal(gx.cpu().numpy(), rx)
    assert np.array_equal(gx[:, 1].cpu().numpy(), fb[:, 1])  # the empty cluster keeps the fp32 fallback
