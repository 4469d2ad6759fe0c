"""GPU parity of the whole SparsePR layer (top-p route + block-sparse attention +
N8 repair), stage by stage against the oracle fed with the GPU's own upstream
results: map bit-exact, probes bit-exact, attention and final output within
max-abs 2e-2 / cosine 0.999 of the float64 closed form."""

from dataclasses import replace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cos(a, b):
    a = a.reshape(-1).astype(np.float64)
    b = b.reshape(-1).astype(np.float64)
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-30))


CONFIGS = {
    # BASELINE config 1 shape (2 heads x 4 frames x 32 x 32, D=64), bf16 on the GPU;
    # 64 probes > 32 q-clusters exercises the representative rounds.
    "c1": dict(shape=("CPU_SMALL", dict(amp=1.0, step_std=0.0, noise_std=0.3)),
               cfg=dict(num_q_centroids=32, num_k_centroids=64, kmeans_iters=10, top_p=0.9, probe_rows=64)),
    # HunyuanVideo-like head layout at a reduced token count (2 heads, 2 x 64 x 64, D=128).
    "small128": dict(shape=("custom", dict(amp=0.3, step_std=0.1, noise_std=0.3)),
                     cfg=dict(num_q_centroids=64, num_k_centroids=128, kmeans_iters=5, top_p=0.9, probe_rows=64)),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_layer_stagewise_parity(dev, oracle, name):
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig

    spec = CONFIGS[name]
    shape_name, gen = spec["shape"]
    shape = synthetic.CPU_SMALL if shape_name == "CPU_SMALL" else synthetic.VideoShape(
        heads=2, frames=2, height=64, width=64, dim=128, components=40)
    q, k, v = synthetic.frame_gmm_qkv(shape, seed=1, device=dev, **gen)
    cfg = SparsePRConfig(**spec["cfg"])
    layer = SparsePRAttention(cfg)
    out = layer(q, k, v)
    route = layer.last_route
    B, H, N, D = q.shape
    qn = q[0].float().cpu().numpy()
    kn = k[0].float().cpu().numpy()
    vn = v[0].float().cpu().numpy()
    ql = route.q_labels.cpu().numpy()
    kl = route.k_labels.cpu().numpy()
    qs = route.q_cluster_sizes.cpu().numpy()
    ks = route.k_cluster_sizes.cpu().numpy()

    # k-means outputs are self-consistent: sizes = counts, fp32 centers = means of the labels
    assert (qs == np.stack([np.bincount(r, minlength=cfg.num_q_centroids) for r in ql])).all()
    assert (ks == np.stack([np.bincount(r, minlength=cfg.num_k_centroids) for r in kl])).all()
    _, mean32, _ = oracle.centroid_update(qn, ql, np.zeros((H, cfg.num_q_centroids, D), np.float32), False)
    nz = qs > 0
    assert (route.q_role_centers.cpu().numpy()[nz] == mean32[nz]).all()

    # top-p map: bit-exact given the GPU centroids
    qc_g, kc_g = (c.float().cpu().numpy() for c in layer.last_centroids)
    nz_k = ks > 0
    assert (qc_g[nz] == oracle.to_bf16(mean32)[nz]).all()
    _, kmean32, _ = oracle.centroid_update(kn, kl, np.zeros((H, cfg.num_k_centroids, D), np.float32), False)
    assert (kc_g[nz_k] == oracle.to_bf16(kmean32)[nz_k]).all()
    gpu_map = route.video_dynamic_map.cpu().numpy()
    ref_map = oracle.identify_dynamic_map(qc_g, kc_g, ks, cfg.top_p, bf16=True)
    assert (gpu_map == ref_map).all()

    # block-sparse attention (before repair) vs the float64 closed form in original token order
    mask = np.stack([gpu_map[h][ql[h]][:, kl[h]] for h in range(H)])
    s = np.einsum("hnd,hmd->hnm", qn.astype(np.float64), kn.astype(np.float64)) / np.sqrt(D)
    s = np.where(mask, s, -np.inf)
    mx = s.max(-1, keepdims=True)
    e = np.where(mask, np.exp(s - np.where(np.isfinite(mx), mx, 0)), 0.0)
    ref_base = np.einsum("hnm,hmd->hnd", e, vn.astype(np.float64)) / np.maximum(e.sum(-1, keepdims=True), 1e-300)
    del s, e
    cfg_norepair = SparsePRConfig(**{**spec["cfg"], "repair": False})
    base_gpu = SparsePRAttention(cfg_norepair)(q, k, v)[0].float().cpu().numpy()
    assert np.abs(base_gpu - ref_base).max() <= 2e-2 and _cos(base_gpu, ref_base) >= 0.999

    # probes: bit-exact rows from the same labels
    rows = route.probe_rows.cpu().numpy()
    if cfg.probe_rows <= cfg.num_q_centroids:
        rr, rw = oracle.select_role_equal_probes_vectorized(qn, ql, cfg.num_q_centroids, cfg.probe_rows)
    else:
        rr, rw = oracle.select_role_equal_probes(qn, ql, cfg.num_q_centroids, cfg.probe_rows)
    assert (rows == rr).all()
    assert np.allclose(route.probe_weights.cpu().numpy(), rw, rtol=1e-6)

    # repair: dense probes, fit, apply, exact scatter vs the oracle on the GPU's base
    dense = oracle.to_bf16(oracle.dense_attention(np.take_along_axis(qn, rr[..., None], 1), kn, vn)
                           .astype(np.float32))
    xfit = np.take_along_axis(base_gpu, rr[..., None], 1)
    # the reference GPU's route: 64 probes at D = 128 take the top-16 subspace basis
    top16 = (cfg.probe_rows, D) == (64, 128)
    state = oracle.fit_reduced_rank_residual(xfit, dense - xfit, 16, 0.1, rw, output_basis_backend="skinny",
                                             decomposition_backend="triton_top16" if top16 else "eigh")
    ref_out = oracle.repair_apply(base_gpu, *state, 1.0, 0.0)
    for h in range(H):
        ref_out[h, rr[h]] = dense[h]
    got = out[0].float().cpu().numpy()
    assert np.abs(got - ref_out).max() <= 2e-2 and _cos(got, ref_out) >= 0.999
    for h in range(H):
        assert np.abs(got[h, rr[h]] - dense[h]).max() <= 1e-2  # probe rows carry the dense output
    info = layer.last_repair_info
    assert 0.0 < float(info["effective_video_density"]) <= 1.0


def test_side_stream_route_matches_one_stream(dev):
    """Q's k-means and the repair's probe part on a side stream give the same bits as
    the whole layer on one stream, on two calls in a row (the second reuses the side
    stream and the allocator's blocks)."""
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig

    shape = synthetic.VideoShape(heads=3, frames=2, height=48, width=64, dim=128, components=40)
    q, k, v = synthetic.frame_gmm_qkv(shape, seed=4, device=dev, amp=1.5, qk_corr=0.3)
    base = dict(num_q_centroids=48, num_k_centroids=96, kmeans_iters=4, top_p=0.85, probe_rows=48)
    one = SparsePRAttention(SparsePRConfig(**base, overlap_streams=False))
    two = SparsePRAttention(SparsePRConfig(**base, overlap_streams=True))
    for call in range(2):
        ref = one(q, k, v)
        out = two(q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {call}: outputs differ"
        assert torch.equal(two.last_route.probe_rows, one.last_route.probe_rows)
        assert torch.equal(two.last_route.video_dynamic_map, one.last_route.video_dynamic_map)


def test_repeated_probe_token_gets_identical_dense_rows(dev):
    """BASELINE config 1's route offers head 1's token 1498 twice as a probe (64 probes over
    32 q-clusters take several representative rounds, and an exhausted group offers its
    token again).  Both copies sit in different waves of the dense probe attention (8 key
    splits of 512 keys).  A row's running maximum moves only on its own growth, so the two
    copies get the same bits, the exact-probe scatter writes one value, and repeated layer
    calls give the same output."""
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig

    q, k, v = synthetic.frame_gmm_qkv(synthetic.CPU_SMALL, seed=0, amp=1.0, step_std=0.0, noise_std=0.3,
                                      qk_corr=1.0, device=dev)
    layer = SparsePRAttention(SparsePRConfig(num_q_centroids=32, num_k_centroids=64, kmeans_iters=10, top_p=0.9,
                                             probe_rows=64))
    route, _ = layer.route(q, k, v)
    rows, _, dense, _ = layer.n8.repair_probes(q, k, v, route)
    torch.cuda.synchronize()
    repeated = 0
    for h in range(rows.shape[0]):
        pos: dict = {}
        for j, t in enumerate(rows[h].tolist()):
            pos.setdefault(t, []).append(j)
        for t, js in pos.items():
            for j in js[1:]:
                repeated += 1
                assert torch.equal(dense[h, j], dense[h, js[0]]), f"head {h} token {t}: probes {js} differ"
    assert repeated > 0, "the configuration no longer repeats a probe token; pick another that does"
    first = layer(q, k, v).clone()
    for _ in range(4):
        assert torch.equal(layer(q, k, v), first)


@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("name", ["c1", "d128"])
def test_graph_replay_matches_eager(dev, name, overlap):
    """The layer captured as a HIP graph gives, on every replay with new inputs, the bits
    of an eager layer (on one stream) fed the same sequence of inputs; eager work and
    synchronisations run between the replays, and the second half of the replays run after
    an eager call of the graphed layer itself.  overlap_streams is set explicitly, so the
    captured side-stream fork and join (Q's k-means and the probe part on the second
    stream) is compared as well as the one-stream capture."""
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig

    if name == "c1":
        shape = synthetic.CPU_SMALL
        cfg = SparsePRConfig(num_q_centroids=32, num_k_centroids=64, kmeans_iters=10, top_p=0.9, probe_rows=64,
                             overlap_streams=overlap)
        gen = dict(amp=1.0, step_std=0.0, noise_std=0.3, qk_corr=1.0)
    else:
        shape = synthetic.VideoShape(heads=3, frames=2, height=48, width=64, dim=128, components=40)
        cfg = SparsePRConfig(num_q_centroids=48, num_k_centroids=96, kmeans_iters=4, top_p=0.85, probe_rows=48,
                             overlap_streams=overlap)
        gen = dict(amp=1.5, qk_corr=0.3)
    inputs = [synthetic.frame_gmm_qkv(shape, seed=s, device=dev, **gen) for s in range(6)]
    graphed_layer = SparsePRAttention(cfg)
    g = graphed_layer.graphed(*inputs[0])
    eager = SparsePRAttention(replace(cfg, overlap_streams=False))
    for _ in range(3):  # the graphed layer's warm-up and capture calls
        eager(*inputs[0])
    for i, (q, k, v) in enumerate(inputs[1:], start=1):
        got = g(q, k, v).clone()
        torch.cuda.synchronize()
        ref = eager(q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {i} differs from the eager call"
        if i == 3:  # an eager call of the graphed layer between replays
            assert torch.equal(graphed_layer(q, k, v), eager(q, k, v))
