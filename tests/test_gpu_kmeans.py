"""GPU parity: k-means assign (bf16 MFMA), segmented centroid mean, Lloyd loop,
exact-FP32 role step.  Labels: identical except ties within 1e-6 of the fp32
distance scale; centroids: bit-exact given identical labels (fp64 sums)."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

TIE_REL = 1e-6


def _gmm(oracle, rng, b, n, d, comps, std=0.25):
    means = rng.standard_normal((b, comps, d)).astype(np.float32)
    which = rng.integers(0, comps, (b, n))
    x = np.take_along_axis(means, which[..., None], 1) + std * rng.standard_normal((b, n, d)).astype(np.float32)
    return oracle.to_bf16(x.astype(np.float32))


@pytest.mark.parametrize("b,n,k,d", [(2, 3000, 256, 128), (3, 1001, 100, 128), (1, 4096, 64, 64),
                                     (2, 500, 512, 128), (1, 37, 5, 64),
                                     (1, 3000, 1000, 128)])  # k > 512: the streamed (non-resident) kernel
@pytest.mark.parametrize("mode", ["bf16", "fp32"])
def test_assign_matches_oracle_up_to_ties(dev, oracle, b, n, k, d, mode):
    from sparsepr_amd.flash_kmeans.kmeans_impl import X_SQ_BF16, X_SQ_FP32, euclid_assign

    rng = np.random.default_rng(n + k + d)
    x = _gmm(oracle, rng, b, n, d, max(k // 2, 2))
    c = oracle.first_k_init(x, k, seed=1)
    labels = euclid_assign(to_dev(x, dev, torch.bfloat16), to_dev(c, dev, torch.bfloat16),
                           x_sq_mode=X_SQ_BF16 if mode == "bf16" else X_SQ_FP32).cpu().numpy()
    x_sq = oracle.x_sq_for(x, mode)
    ref, dist = oracle.kmeans_assign(x, c, x_sq)
    ok, nbad = oracle.label_mismatches_are_ties(labels, ref, dist, x_sq, c, TIE_REL)
    assert ok, f"{nbad} label mismatches beyond tie tolerance"
    assert nbad <= max(2, labels.size // 1000)


def test_assign_planted_exact_ties_pick_lowest_index(dev, oracle):
    from sparsepr_amd.flash_kmeans.kmeans_impl import euclid_assign

    rng = np.random.default_rng(3)
    c = oracle.to_bf16(rng.standard_normal((1, 200, 128)).astype(np.float32))
    c[0, 150] = c[0, 7]   # duplicate across LDS tiles
    c[0, 40] = c[0, 33]   # duplicate within a tile
    x = np.repeat(c[:, [7, 33, 150, 40]], 70, axis=1)  # points exactly on the centroids
    labels = euclid_assign(to_dev(x, dev, torch.bfloat16), to_dev(c, dev, torch.bfloat16)).cpu().numpy()
    assert (labels[0, :70] == 7).all() and (labels[0, 70:140] == 33).all()
    assert (labels[0, 140:210] == 7).all() and (labels[0, 210:] == 33).all()


def test_assign_with_given_x_sq(dev, oracle):
    from sparsepr_amd.flash_kmeans import euclid_assign_triton

    rng = np.random.default_rng(4)
    x = _gmm(oracle, rng, 2, 2000, 128, 40)
    c = oracle.first_k_init(x, 64, seed=2)
    xt = to_dev(x, dev, torch.bfloat16)
    x_sq = (xt.float() ** 2).sum(-1)
    labels = euclid_assign_triton(xt, to_dev(c, dev, torch.bfloat16), x_sq).cpu().numpy()
    xs = oracle.x_sq_for(x, "fp32")
    ref, dist = oracle.kmeans_assign(x, c, xs)
    ok, _ = oracle.label_mismatches_are_ties(labels, ref, dist, xs, c, TIE_REL)
    assert ok


@pytest.mark.parametrize("k,d", [(256, 128), (7, 64), (512, 128), (2, 128), (5, 128)])  # k <= 7: split clusters
def test_centroid_mean_bit_exact(dev, oracle, k, d):
    from sparsepr_amd.flash_kmeans.kmeans_impl import centroid_update_sorted

    rng = np.random.default_rng(k)
    n = 5000
    x = _gmm(oracle, rng, 2, n, d, 30)
    labels = rng.integers(0, k, (2, n)).astype(np.int32)
    labels[labels == 3] = 4  # cluster 3 empty
    old = oracle.to_bf16(rng.standard_normal((2, k, d)).astype(np.float32))
    res = centroid_update_sorted(to_dev(x, dev, torch.bfloat16), to_dev(labels, dev),
                                 to_dev(old, dev, torch.bfloat16), want_mean32=True, want_shift=True)
    cent, mean32, counts = oracle.centroid_update(x, labels, old, out_bf16=True)
    assert (res.mean32.cpu().numpy() == mean32).all()
    assert (res.centroids.float().cpu().numpy() == cent).all()
    assert (res.sizes.cpu().numpy() == counts).all()
    shift = np.sqrt(((cent.astype(np.float64) - old) ** 2).sum(-1)).max()
    assert abs(float(res.shift.item()) - shift) <= 1e-5 * max(shift, 1.0)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 48)])
def test_centroid_mean_skewed_clusters(dev, oracle, dtype, d):
    """Each cluster's rows are cut into 512-row slices planned on the device: one cluster holds
    about 80 % of the rows (dozens of slices, summed by the finalize kernel), one about 5 %
    (a few slices), the rest one slice each (finalized by that slice's workgroup), two none
    (the previous centroid): every mean bit-exact to the float64 one."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import centroid_update_sorted

    rng = np.random.default_rng(41 + d)
    b, n, k = 2, 30000, 40
    x = _gmm(oracle, rng, b, n, d, 20)
    if dtype == torch.float32:
        x = (x + 1e-3 * rng.standard_normal(x.shape)).astype(np.float32)  # not bf16 values
    labels = rng.integers(8, k, (b, n)).astype(np.int32)
    u = rng.random((b, n))
    labels[u < 0.8] = 0
    labels[(u >= 0.8) & (u < 0.85)] = 7
    old = rng.standard_normal((b, k, d)).astype(np.float32)
    if dtype == torch.bfloat16:
        old = oracle.to_bf16(old)
    res = centroid_update_sorted(to_dev(x, dev, dtype), to_dev(labels, dev), to_dev(old, dev, dtype),
                                 want_mean32=True, want_shift=True)
    cent, mean32, counts = oracle.centroid_update(x, labels, old, out_bf16=dtype == torch.bfloat16)
    assert counts[0, 0] > 40 * 512 and counts[0, 5] == 0 and counts[0, 6] == 0
    assert (res.mean32.cpu().numpy() == mean32).all()
    assert (res.centroids.float().cpu().numpy() == cent).all()
    assert (res.sizes.cpu().numpy() == counts).all()


def test_centroid_update_accumulates_into_buffers(dev, oracle):
    from sparsepr_amd.flash_kmeans import triton_centroid_update_sorted_euclid

    rng = np.random.default_rng(9)
    x = _gmm(oracle, rng, 1, 800, 128, 10)
    labels = rng.integers(0, 16, (1, 800)).astype(np.int32)
    old = oracle.to_bf16(rng.standard_normal((1, 16, 128)).astype(np.float32))
    sums = torch.ones((1, 16, 128), dtype=torch.float32, device=dev)
    cnts = torch.full((1, 16), 2, dtype=torch.int32, device=dev)
    out = triton_centroid_update_sorted_euclid(to_dev(x, dev, torch.bfloat16), to_dev(labels, dev),
                                               to_dev(old, dev, torch.bfloat16), centroid_sums=sums,
                                               centroid_cnts=cnts, calculate_new=False)
    assert out is None
    ref_sums = np.zeros((16, 128))
    np.add.at(ref_sums, labels[0], x[0].astype(np.float64))
    assert np.allclose(sums[0].cpu().numpy(), 1.0 + ref_sums, rtol=1e-6, atol=1e-5)
    assert (cnts[0].cpu().numpy() == 2 + np.bincount(labels[0], minlength=16)).all()


def test_lloyd_stepwise_parity(dev, oracle):
    """Each iteration: GPU labels == oracle labels up to ties; given the GPU's
    labels, the GPU centroids equal the oracle's bit for bit."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import X_SQ_BF16, centroid_update_sorted, euclid_assign

    rng = np.random.default_rng(11)
    x = _gmm(oracle, rng, 3, 6000, 128, 100)
    xt = to_dev(x, dev, torch.bfloat16)
    cent = oracle.first_k_init(x, 128, seed=3)
    x_sq = oracle.x_sq_for(x, "bf16")
    for _ in range(5):
        ct = to_dev(cent, dev, torch.bfloat16)
        lab = euclid_assign(xt, ct, x_sq_mode=X_SQ_BF16).cpu().numpy()
        ref, dist = oracle.kmeans_assign(x, cent, x_sq)
        ok, _ = oracle.label_mismatches_are_ties(lab, ref, dist, x_sq, cent, TIE_REL)
        assert ok
        res = centroid_update_sorted(xt, to_dev(lab, dev), ct)
        new, _, counts = oracle.centroid_update(x, lab, cent, out_bf16=True)
        assert (res.centroids.float().cpu().numpy() == new).all()
        assert (res.sizes.cpu().numpy() == counts).all()
        cent = new


def test_batch_kmeans_euclid_whole_loop(dev, oracle):
    from sparsepr_amd.flash_kmeans import batch_kmeans_Euclid

    rng = np.random.default_rng(12)
    x = _gmm(oracle, rng, 2, 4000, 128, 60)
    init = oracle.first_k_init(x, 64, seed=4)
    labels, cent, iters = batch_kmeans_Euclid(to_dev(x, dev, torch.bfloat16), 64, max_iters=5,
                                              init_centroids=to_dev(init, dev, torch.bfloat16))
    rl, rc, rs, ri = oracle.batch_kmeans_euclid(x, 64, 5, 0.0, init, "bf16", True)
    assert iters == ri == 5
    agree = (labels.cpu().numpy() == rl).mean()
    assert agree > 0.999
    if agree == 1.0:
        assert (cent.float().cpu().numpy() == rc).all()
    # tol larger than any shift: stops after one iteration and returns the init
    labels, cent, iters = batch_kmeans_Euclid(to_dev(x, dev, torch.bfloat16), 64, max_iters=5, tol=1e9,
                                              init_centroids=to_dev(init, dev, torch.bfloat16))
    assert iters == 1 and (cent.float().cpu().numpy() == init).all()


@pytest.mark.parametrize("backend,x_sq_mode,labels_dtype,sizes_dtype", [
    ("cuvs", "bf16", torch.int64, torch.int32),   # in-file loop: x.dtype x_sq buffer (kmeans_utils.py:1550-1580)
    ("flash", "fp32", torch.int32, torch.int64),  # warm start: inline fp32 x_sq (kmeans_utils.py:1396-1411)
])
def test_kmeans_utils_dispatcher_warm_start(dev, oracle, backend, x_sq_mode, labels_dtype, sizes_dtype):
    """kmeans_utils.batch_kmeans_Euclid (:1504-1580) at its default tol = 1e-4, warm
    started, against the oracle's loop with that backend's x_sq precision."""
    from sparsepr_amd.kmeans_utils import batch_kmeans_Euclid

    rng = np.random.default_rng(17)
    x = _gmm(oracle, rng, 2, 4000, 128, 60)
    init = oracle.first_k_init(x, 64, seed=5)
    labels, cent, sizes, iters = batch_kmeans_Euclid(to_dev(x, dev, torch.bfloat16), 64, max_iters=4,
                                                     init_centroids=to_dev(init, dev, torch.bfloat16),
                                                     backend=backend)
    rl, rc, rs, ri = oracle.batch_kmeans_euclid(x, 64, 4, 1e-4, init, x_sq_mode, True)
    assert labels.dtype == labels_dtype and sizes.dtype == sizes_dtype
    assert iters == ri
    agree = (labels.cpu().numpy() == rl).mean()
    assert agree > 0.999
    if agree == 1.0:
        assert (cent.float().cpu().numpy() == rc).all()
        assert (sizes.cpu().numpy() == rs).all()
    # points sitting exactly on the initial centroids converge at once: shift 0 < tol
    x0 = np.repeat(init, 10, axis=1)
    labels, cent, sizes, iters = batch_kmeans_Euclid(to_dev(x0, dev, torch.bfloat16), 64, max_iters=4,
                                                     init_centroids=to_dev(init, dev, torch.bfloat16),
                                                     backend=backend)
    assert iters == 1 and (cent.float().cpu().numpy() == init).all()
    assert (sizes.cpu().numpy() == 10).all()


@pytest.mark.parametrize("backend", ["cuvs", "flash"])
def test_kmeans_utils_assign_only(dev, oracle, backend):
    """max_iters = 0 (kmeans_utils.py:1212-1278): one assignment to the given centroids
    with the fp32 x_sq, int64 labels and sizes, 0 iterations, centroids unchanged."""
    from sparsepr_amd.kmeans_utils import batch_kmeans_Euclid

    rng = np.random.default_rng(18)
    x = _gmm(oracle, rng, 2, 3000, 128, 40)
    c = oracle.first_k_init(x, 100, seed=6)
    ct = to_dev(c, dev, torch.bfloat16)
    labels, cent, sizes, iters = batch_kmeans_Euclid(to_dev(x, dev, torch.bfloat16), 100, max_iters=0,
                                                     init_centroids=ct, backend=backend)
    assert iters == 0 and labels.dtype == torch.int64 and sizes.dtype == torch.int64
    assert torch.equal(cent, ct)
    xs = oracle.x_sq_for(x, "fp32")
    ref, dist = oracle.kmeans_assign(x, c, xs)
    got = labels.cpu().numpy()
    ok, _ = oracle.label_mismatches_are_ties(got, ref, dist, xs, c, TIE_REL)
    assert ok
    assert (sizes.cpu().numpy() == np.stack([np.bincount(r, minlength=100) for r in got])).all()
    with pytest.raises(RuntimeError, match="requires init_centroids"):
        batch_kmeans_Euclid(to_dev(x, dev, torch.bfloat16), 100, max_iters=0, backend=backend)


def test_kmeans_utils_n8_backend_and_errors(dev, oracle):
    """backend n8_cuda_ext (:1468-1501): fixed exact-FP32 D = 64 steps from given centroids."""
    from sparsepr_amd.kmeans_utils import batch_kmeans_Euclid

    rng = np.random.default_rng(19)
    f = rng.standard_normal((2, 2000, 64)).astype(np.float32)
    c = f[:, :40].copy()
    labels, cent, sizes, iters = batch_kmeans_Euclid(to_dev(f, dev), 40, max_iters=2, init_centroids=to_dev(c, dev),
                                                     backend="n8_cuda_ext")
    l1, c1, _, _ = oracle.role_step64(f, c)
    l2, c2, s2, _ = oracle.role_step64(f, c1)
    assert iters == 2 and sizes.dtype == torch.int64
    assert (labels.cpu().numpy() == l2).mean() > 0.999
    with pytest.raises(RuntimeError, match="Unknown Euclidean k-means backend"):
        batch_kmeans_Euclid(to_dev(f, dev), 40, backend="bogus")
    with pytest.raises(RuntimeError, match="requires initialized centroids"):
        batch_kmeans_Euclid(to_dev(f, dev), 40, max_iters=2, backend="n8_cuda_ext")


def test_kmeans_full_size_properties(dev):
    """BASELINE config 2 shape (24 x 118,800 x 128, K=256, 5 iterations):
    sizes sum to N, the objective does not increase, labels are the argmin."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import X_SQ_BF16, euclid_assign, lloyd

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    b, n, d, k = 24, 118800, 128, 256
    means = torch.randn(b, k, d, device=dev, generator=g)
    which = torch.randint(0, k, (b, n), device=dev, generator=g)
    x = (torch.gather(means, 1, which[..., None].expand(-1, -1, d))
         + 0.25 * torch.randn(b, n, d, device=dev, generator=g)).to(torch.bfloat16)
    init = x[:, torch.randperm(n, device=dev, generator=g)[:k]]
    res = lloyd(x, k, 5, 0.0, init, x_sq_mode=X_SQ_BF16)
    assert bool((res.sizes.sum(1) == n).all())
    xf = x.float()

    def objective(c):
        lab = euclid_assign(x, c, x_sq_mode=X_SQ_BF16).long()
        return ((xf - torch.gather(c.float(), 1, lab[..., None].expand(-1, -1, d))) ** 2).sum().item()

    assert objective(res.centroids) <= objective(init) * 1.0001
    # spot-check argmin on a slice against a float64 evaluation
    lab = euclid_assign(x, res.centroids, x_sq_mode=X_SQ_BF16)[:2, :2000].long()
    dd = torch.cdist(xf[:2, :2000].double(), res.centroids[:2].double())
    best = dd.gather(2, lab[..., None])[..., 0]
    assert bool(((best - dd.min(2).values) <= 1e-3 * dd.min(2).values + 1e-3).all())


@pytest.mark.parametrize("b,n,k,d", [(2, 3000, 300, 64), (2, 2500, 1000, 48), (1, 777, 37, 16), (1, 1000, 64, 32),
                                     (1, 600, 70, 128), (3, 2100, 77, 48), (3, 1900, 77, 48), (3, 1900, 120, 64),
                                     (2, 1500, 600, 128)])
def test_assign_tf32_matches_oracle_up_to_ties(dev, oracle, b, n, k, d):
    """fp32 role-space features (the N8 route's shapes: rank 64 / 300 Q clusters, rank 48 /
    1000 K clusters): TF32 products, fp32 norms, lowest index on ties.  (3, 1900, 77, 48)
    and (3, 1900, 120, 64) give the resident kernel (12 waves per workgroup at these D)
    workgroups whose shares of 64-point blocks cross from one batch into the next (30 blocks
    per batch, 8 workgroups of 11.25 blocks); (2, 1500, 600, 128) does not fit its LDS and
    runs the streamed kernel."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import euclid_assign

    rng = np.random.default_rng(n + k + d)
    means = rng.standard_normal((b, max(k // 3, 2), d)).astype(np.float32)
    x = (means[:, rng.integers(0, means.shape[1], n)] + 0.3 * rng.standard_normal((b, n, d))).astype(np.float32)
    c = x[:, rng.permutation(n)[:k]].copy()
    c[:, k // 2] = c[:, 1]  # an exact duplicate: the lower index wins
    x_sq_out = torch.empty((b, n), device=dev)
    labels = euclid_assign(to_dev(x, dev), to_dev(c, dev), x_sq_out=x_sq_out).cpu().numpy()
    ref, dist, x_sq = oracle.kmeans_assign_tf32(x, c)
    ok, nbad = oracle.label_mismatches_are_ties(labels, ref, dist, x_sq, c, TIE_REL)
    assert ok, f"{nbad} label mismatches beyond tie tolerance"
    assert nbad <= max(2, labels.size // 1000)
    assert (labels != k // 2).all()
    assert np.allclose(x_sq_out.cpu().numpy(), x_sq, rtol=1e-6)


@pytest.mark.parametrize("d", [48, 64])
def test_assign_tf32_wide_range(dev, oracle, d):
    """The TF32 products go through fp16 images scaled by a power of two per point row and per
    64-centroid tile: rows and centroids spread over 10^-3 .. 10^5 (past fp16's 65504 and below
    its normal range without the scale), with tiny entries inside rows, still match the oracle's
    TF32 assignment up to ties."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import euclid_assign

    rng = np.random.default_rng(d + 5)
    b, n, k = 2, 2000, 300
    cmag = 10.0 ** rng.uniform(-3, 5, (b, k, 1))
    c = (rng.standard_normal((b, k, d)) * cmag).astype(np.float32)
    pick = rng.integers(0, k, (b, n))
    x = np.take_along_axis(c, pick[..., None], 1) * (1 + 0.05 * rng.standard_normal((b, n, d)))
    x[:, ::7, 3] *= 1e-6  # entries far below their row's largest one
    x = x.astype(np.float32)
    labels = euclid_assign(to_dev(x, dev), to_dev(c, dev)).cpu().numpy()
    ref, dist, x_sq = oracle.kmeans_assign_tf32(x, c)
    ok, nbad = oracle.label_mismatches_are_ties(labels, ref, dist, x_sq, c, TIE_REL)
    assert ok, f"{nbad} label mismatches beyond tie tolerance"
    assert nbad <= max(2, labels.size // 1000)


def test_lloyd_fp32_features_tf32(dev, oracle):
    """The flash Lloyd loop on fp32 features, one iteration at a time: each iteration's labels
    against the oracle's TF32 assignment from the same centroids, centroids the means."""
    from sparsepr_amd.flash_kmeans.kmeans_impl import lloyd

    rng = np.random.default_rng(23)
    b, n, d, k = 2, 4000, 48, 200
    means = rng.standard_normal((b, 60, d)).astype(np.float32)
    x = (means[:, rng.integers(0, 60, n)] + 0.3 * rng.standard_normal((b, n, d))).astype(np.float32)
    c = x[:, :k].copy()
    xt = to_dev(x, dev)
    cent = to_dev(c, dev)
    for it in range(3):
        res = lloyd(xt, k, 1, 0.0, cent)
        ref, dist, x_sq = oracle.kmeans_assign_tf32(x, cent.cpu().numpy())
        got = res.labels.cpu().numpy()
        ok, nbad = oracle.label_mismatches_are_ties(got, ref, dist, x_sq, cent.cpu().numpy(), TIE_REL)
        assert ok and nbad <= 2
        new, mean32, _ = oracle.centroid_update(x, got, cent.cpu().numpy(), out_bf16=False)
        # fp64 sums of fp32 rows: equal up to the last fp64 bit, so up to rare fp32 double rounding
        assert np.allclose(res.centroids.cpu().numpy(), new, rtol=1e-6, atol=1e-7)
        cent = res.centroids


def test_role_step64_exact(dev, oracle):
    from sparsepr_amd.kernels.n8_extension import role_cluster_step_k64, role_cluster_step_q64

    rng = np.random.default_rng(13)
    f = rng.standard_normal((2, 3000, 64)).astype(np.float32)
    c = rng.standard_normal((2, 300, 64)).astype(np.float32)
    c[:, 250] = c[:, 17]
    labels, cent, sizes = role_cluster_step_q64(to_dev(f, dev), to_dev(c, dev))
    rl, rc, rs, _ = oracle.role_step64(f, c)
    assert (labels.cpu().numpy() == rl).all()
    assert (sizes.cpu().numpy() == rs).all()
    assert np.allclose(cent.cpu().numpy(), rc, rtol=1e-5, atol=1e-6)
    c2 = rng.standard_normal((2, 1000, 64)).astype(np.float32)
    labels, cent, sizes = role_cluster_step_k64(to_dev(f, dev), to_dev(c2, dev))
    rl, rc, rs, _ = oracle.role_step64(f, c2)
    assert (labels.cpu().numpy() == rl).all()
    with pytest.raises(RuntimeError):
        role_cluster_step_q64(to_dev(f, dev), to_dev(c2, dev))  # 1000 > 512 clusters
