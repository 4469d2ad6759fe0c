"""GPU parity of the native N8V6Core.route (n8_v6.py:521-1172), stage by stage, each stage
against the oracle fed with the GPU's own upstream tensors (captured through the route's
diagnostic callback), over a cold call and a warm call; then route + block-sparse attention
+ repair in the HunyuanVideo adapter's composition (video tokens + a text suffix, the full
K/V layout, hunyuanvideo.py:160-239) at the default N8 configuration.

Tolerances: metrics 1e-5 relative (fp32 sums); factors through F F^T 1e-3 (eigengap-limited);
labels equal to the oracle's TF32 assignment up to ties (1e-6); centroids exact (fp64 sums
of bf16 rows) or 1e-6 (fp32 role features); selector maps bit-exact given the GPU scores;
attention and repaired outputs max-abs 2e-2 / cosine 0.999."""

import math

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

TIE_REL = 1e-6


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _gram(f):
    f = np.asarray(f, np.float64)
    return np.einsum("bir,bjr->bij", f, f)


def _inputs(dev, heads=2, frames=2, h=64, w=64, seed=7):
    from sparsepr_amd import synthetic

    shape = synthetic.VideoShape(heads=heads, frames=frames, height=h, width=w, dim=128, components=60)
    return synthetic.frame_gmm_qkv(shape, seed=seed, device=dev, amp=2.3, qk_corr=0.3, step_std=0.1,
                                   noise_std=0.3)


class _Capture:
    def __init__(self):
        self.items = []

    def __call__(self, stage, tensors, scalars):
        self.items.append((stage, {k: v.detach().clone() for k, v in tensors.items()}, dict(scalars)))

    def get(self, name):
        for _, tensors, _ in self.items:
            if name in tensors:
                return tensors[name]
        raise KeyError(name)


def _check_scores(scores, ref):
    """Scores are logs of value errors (or masses) E.  With exact centroids a singleton or
    constant cluster has E at the rounding floor, where the log is ill-conditioned; so E is
    compared relative to the row's largest E (2e-3), and the log only where E is within three
    decades of it (2e-3)."""
    fin = np.isfinite(ref)
    assert (np.isfinite(scores) == fin).all()
    row_max = np.where(fin, ref, -np.inf).max(-1, keepdims=True)
    e_ref = np.where(fin, np.exp(ref - row_max), 0.0)
    e_got = np.where(fin, np.exp(scores.astype(np.float64) - row_max), 0.0)
    assert np.abs(e_got - e_ref).max() <= 2e-3
    big = fin & (ref - row_max > -3 * np.log(10.0))
    assert np.abs(scores[big] - ref[big]).max() <= 2e-3


def _check_warm_factor(got, ref, cfg):
    """Warm factors entry by entry (2e-3 of the largest entry); the full Rayleigh-Ritz finish
    has the eigensolver's column signs, so it is compared through F F^T (1e-4 relative)."""
    if cfg.factor_ritz_mode == "full":
        assert _rel(_gram(got), _gram(ref)) <= 1e-4
    else:
        assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max()


def _check_call(oracle, core, q, k, v, cap, route, cfg, prev=None):
    """Stagewise checks of one route call.  prev: the state before the call (warm calls)."""
    from sparsepr_amd import operator_kmeans as ok
    from sparsepr_amd.kernels.role_projection import role_k_projection_normalize, role_kv_projection_normalize

    B, H, N, D = q.shape
    qf = q.reshape(H, N, D)
    kf = k.reshape(H, N, D)
    vf = v.reshape(H, N, D)
    qn, kn, vn = (t.float().cpu().numpy() for t in (qf, kf, vf))
    # K metric: the uncentred second moment of the deterministic Q sample
    k_metric = cap.get("k_role_metric")
    pos = ok.deterministic_token_positions(N, cfg.metric_sample_tokens, q.device).cpu().numpy()
    assert _rel(k_metric.cpu().numpy(), oracle.role_metric(qn, rows=pos)) <= 1e-5
    # K factor: cold eigen factor, or one warm subspace update from the previous state
    kfac = core.k_factor_current.cpu().numpy()
    if prev is None:
        assert _rel(_gram(kfac), _gram(oracle.metric_factor(k_metric.cpu().numpy(), cfg.role_k_rank))) <= 1e-3
    else:
        rf, rb, rrec = oracle.warm_subspace_metric_factor(
            k_metric.cpu().numpy(), prev["k_state"], cfg.role_k_rank, cfg.factor_power_iters,
            cfg.factor_orthogonalization, cfg.factor_ritz_mode, cfg.factor_rayleigh_ridge,
            cfg.factor_cholesky_qr_ridge)
        assert not rrec.any() and not core.k_factor_recovery_mask.any()
        _check_warm_factor(kfac, rf, cfg)
    joint = cfg.role_v_weight > 0.0
    precision = cfg.role_kv_matmul_precision if cfg.compile_role_kv_projection else "highest"
    if joint:
        # V metric: the centred covariance of the deterministic V sample, and the V factor
        v_metric = cap.get("v_role_metric")
        assert _rel(v_metric.cpu().numpy(), oracle.role_metric(vn, rows=pos, center=True)) <= 1e-5
        vfac = core.v_factor_current.cpu().numpy()
        if prev is None:
            assert _rel(_gram(vfac), _gram(oracle.metric_factor(v_metric.cpu().numpy(), cfg.role_v_rank))) <= 1e-3
        else:
            rf, rb, rrec = oracle.warm_subspace_metric_factor(
                v_metric.cpu().numpy(), prev["v_state"], cfg.role_v_rank, cfg.factor_power_iters,
                cfg.factor_orthogonalization, cfg.factor_ritz_mode, cfg.factor_rayleigh_ridge,
                cfg.factor_cholesky_qr_ridge)
            assert not rrec.any() and not core.v_factor_recovery_mask.any()
            _check_warm_factor(vfac, rf, cfg)
    # K role features under the K/V matmul precision (joint with the weighted V features) and
    # the K k-means: the final labels are the TF32 argmin of the centroids entering the last
    # iteration, which a GPU Lloyd with one iteration fewer from the route's initialisation
    # reproduces (warm calls)
    if joint:
        kfeat, kscale, vscale = role_kv_projection_normalize(kf, vf, core.k_factor_current, core.v_factor_current,
                                                             cfg.role_v_weight, precision=precision)
        ref_feat = oracle.role_kv_projection_normalize(kn, vn, core.k_factor_current.cpu().numpy(),
                                                       core.v_factor_current.cpu().numpy(), cfg.role_v_weight,
                                                       precision)[0]
    else:
        kfeat, kscale = role_k_projection_normalize(kf, core.k_factor_current, precision=precision)
        ref_feat = oracle.role_k_projection_normalize(kn, core.k_factor_current.cpu().numpy(), precision)[0]
    assert np.abs(kfeat.cpu().numpy().astype(np.float64) - ref_feat).max() <= 2e-5 * max(np.abs(ref_feat).max(), 1)
    klab = route.k_labels.cpu().numpy()
    ksz = route.k_cluster_sizes.cpu().numpy()
    assert (ksz == np.stack([np.bincount(r, minlength=cfg.num_k_centroids) for r in klab])).all()
    if prev is not None:
        from sparsepr_amd.flash_kmeans.kmeans_impl import lloyd
        from sparsepr_amd.kernels.role_metric import project_rows

        kinit = project_rows(prev["k_centroids"], core.k_factor_current, divisor=kscale, precision=precision)
        if joint:
            kinit = torch.cat((kinit, project_rows(prev["v_centroids"], core.v_factor_current, divisor=vscale,
                                                   precision=precision, weight=cfg.role_v_weight)), dim=2)
        iters = route.k_kmeans_iters
        start = kinit if iters == 1 else lloyd(kfeat, cfg.num_k_centroids, iters - 1, 0.0, kinit).centroids
        ref, dist, xsq = oracle.kmeans_assign_tf32(kfeat.cpu().numpy(), start.cpu().numpy())
        ok_, nbad = oracle.label_mismatches_are_ties(klab, ref, dist, xsq, start.cpu().numpy(), TIE_REL)
        assert ok_ and nbad <= 5
    # K and V original-space centroids: exact fp64 means of the bf16 rows (empty -> previous)
    kc_prev = np.zeros((H, cfg.num_k_centroids, D), np.float32) if prev is None else prev["k_centroids_np"]
    vc_prev = np.zeros((H, cfg.num_k_centroids, D), np.float32) if prev is None else prev["v_centroids_np"]
    _, kmean, _ = oracle.centroid_update(kn, klab, kc_prev, out_bf16=False)
    _, vmean, _ = oracle.centroid_update(vn, klab, vc_prev, out_bf16=False)
    assert np.array_equal(core.k_centroids.cpu().numpy(), kmean)
    assert np.array_equal(core.v_centroids.cpu().numpy(), vmean)
    # Q metric from the key centroids, Q factor
    q_metric = cap.get("q_role_metric")
    assert _rel(q_metric.cpu().numpy(), oracle.role_metric(kmean, sizes=ksz, center=True, post_scale=1.0 / D)) <= 1e-5
    if prev is None:
        assert _rel(_gram(core.q_factor_current.cpu().numpy()),
                    _gram(oracle.metric_factor(q_metric.cpu().numpy(), cfg.role_q_rank))) <= 1e-3
    # Q role features: per-row RMS-normalised TF32 projection
    qfeat = route.q_role_features.cpu().numpy()
    ref_qfeat = oracle.role_projection_rms(qn, core.q_factor_current.cpu().numpy())
    assert np.abs(qfeat - ref_qfeat).max() <= 1e-4
    qlab = route.q_labels.cpu().numpy()
    qsz = route.q_cluster_sizes.cpu().numpy()
    assert (qsz == np.stack([np.bincount(r, minlength=cfg.num_q_centroids) for r in qlab])).all()
    qc_prev = np.zeros((H, cfg.num_q_centroids, D), np.float32) if prev is None else prev["q_centroids_np"]
    _, qmean, _ = oracle.centroid_update(qn, qlab, qc_prev, out_bf16=False)
    assert np.array_equal(core.q_centroids.cpu().numpy(), qmean)
    # the K/V permutation: the stable argsort of the labels, rows gathered exactly
    order = route.k_sorted_indices.cpu().numpy()
    assert (order == np.argsort(klab, axis=1, kind="stable")).all()
    # selector scores (SVG-EAR value error) on the permuted K/V, then the exact budget map
    scores = cap.get("svg_ear_scores").cpu().numpy()
    ks_np = route.k_permuted.reshape(H, -1, D).float().cpu().numpy()
    vs_np = route.v_permuted.reshape(H, -1, D).float().cpu().numpy()
    ref_scores = oracle.svg_ear_value_error_scores(qmean, ks_np, vs_np, kmean, vmean, ksz, 1)
    _check_scores(scores, ref_scores)
    budgets = cap.get("requested_key_budget").cpu().numpy()
    want_map = oracle.select_budget(scores, ksz, budgets, mode=1)[:, 1:, 1:]
    assert (route.video_dynamic_map.cpu().numpy() == want_map).all()


def test_n8_route_stagewise_cold_and_warm(dev, oracle):
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    q, k, v = _inputs(dev)
    B, H, N, D = q.shape
    cfg = N8V6Config(num_q_centroids=64, num_k_centroids=200, kmeans_iter_init=6, kmeans_iter_step=2,
                     probe_rows=32, target_density=0.25)
    core = N8V6Core(cfg)
    cap = _Capture()
    core.diagnostic_callback = cap
    route = core.route(q, k, v)
    torch.cuda.synchronize()
    assert route.video_dynamic_map.shape == (H, 64, 200) and route.video_dynamic_map.dtype == torch.bool
    budget = max(0, int(math.ceil(max(0.0, cfg.target_density - cfg.probe_rows / N) * N)))
    assert route.base_video_density == budget / N
    _check_call(oracle, core, q, k, v, cap, route, cfg)
    prev = {"k_state": core.k_factor_state.cpu().numpy(), "k_centroids": core.k_centroids.clone(),
            "k_centroids_np": core.k_centroids.cpu().numpy(), "v_centroids_np": core.v_centroids.cpu().numpy(),
            "q_centroids_np": core.q_centroids.cpu().numpy()}
    # the next denoising step: slightly moved inputs, warm factors and warm k-means
    q2, k2, v2 = (t + (0.05 * torch.randn(t.shape, device=dev)).to(t.dtype) for t in (q, k, v))
    cap2 = _Capture()
    core.diagnostic_callback = cap2
    route2 = core.route(q2, k2, v2)
    torch.cuda.synchronize()
    assert route2.k_kmeans_iters <= cfg.kmeans_iter_step and core.route_call_index == 2
    _check_call(oracle, core, q2, k2, v2, cap2, route2, cfg, prev=prev)


def _state_of(core):
    return {"k_state": core.k_factor_state.cpu().numpy(), "k_centroids": core.k_centroids.clone(),
            "v_state": None if core.v_factor_state is None else core.v_factor_state.cpu().numpy(),
            "v_centroids": core.v_centroids.clone(), "k_centroids_np": core.k_centroids.cpu().numpy(),
            "v_centroids_np": core.v_centroids.cpu().numpy(), "q_centroids_np": core.q_centroids.cpu().numpy()}


@pytest.mark.parametrize("v_weight,precision,compiled,ortho,ritz", [
    (0.5, "high", True, "each_cholesky_qr2", "rayleigh_cholesky"),
    (0.0, "highest", True, "each_cholesky_qr2", "rayleigh_cholesky"),
    (0.0, "medium", True, "each_cholesky_qr2", "rayleigh_cholesky"),
    (0.7, "medium", False, "each_cholesky_qr2", "rayleigh_cholesky"),
    (0.0, "high", False, "each_cholesky_qr2", "rayleigh_cholesky"),
    (0.0, "high", True, "each_qr", "full"),
    (0.5, "high", True, "final_qr", "rayleigh_cholesky")])
def test_n8_route_joint_kv_features_and_precisions(dev, oracle, v_weight, precision, compiled, ortho, ritz):
    """role_v_weight > 0 (the V metric and factor, joint K/V role features for the K k-means,
    n8_v6.py:611-704), the K/V projection precisions (role_kv_matmul_precision; uncompiled
    projections are fp32) and the Householder-QR / full Rayleigh-Ritz warm factor updates
    (factor_orthogonalization, factor_ritz_mode), stage by stage on a cold and a warm call."""
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    q, k, v = _inputs(dev, seed=13)
    cfg = N8V6Config(num_q_centroids=48, num_k_centroids=160, kmeans_iter_init=5, kmeans_iter_step=2,
                     probe_rows=32, target_density=0.25, role_v_weight=v_weight, role_v_rank=16,
                     role_kv_matmul_precision=precision, compile_role_kv_projection=compiled,
                     factor_orthogonalization=ortho, factor_ritz_mode=ritz)
    core = N8V6Core(cfg)
    cap = _Capture()
    core.diagnostic_callback = cap
    route = core.route(q, k, v)
    torch.cuda.synchronize()
    _check_call(oracle, core, q, k, v, cap, route, cfg)
    prev = _state_of(core)
    q2, k2, v2 = (t + (0.05 * torch.randn(t.shape, device=dev)).to(t.dtype) for t in (q, k, v))
    cap2 = _Capture()
    core.diagnostic_callback = cap2
    route2 = core.route(q2, k2, v2)
    torch.cuda.synchronize()
    _check_call(oracle, core, q2, k2, v2, cap2, route2, cfg, prev=prev)


@pytest.mark.parametrize("features,rank", [("output_role", 16), ("output", 32), ("output_role", 64)])
def test_n8_output_role_repair(dev, oracle, features, rank):
    """repair_features "output_role" (n8_v6.py:1246-1371): the fit's features are the base
    output's probe rows and the route's Q role features at those rows (exact), P = 128 + 64
    features on 64 probes (the dual fit; the top-16 basis at rank 16, the exact one at other
    ranks); and repair_rank 32 / 64.  The repaired output against the float64 oracle's fit
    and apply of the same inputs, probe rows exact."""
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    q, k, v = _inputs(dev, seed=17)
    B, H, N, D = q.shape
    cfg = N8V6Config(num_q_centroids=96, num_k_centroids=200, kmeans_iter_init=4, probe_rows=64,
                     target_density=0.25, repair_features=features, repair_rank=rank)
    role_dim = cfg.role_q_rank if features == "output_role" else 0
    core = N8V6Core(cfg)
    route = core.route(q, k, v)
    g = torch.Generator(device=dev).manual_seed(3)
    base = (0.5 * torch.randn(q.shape, device=dev, generator=g)).to(torch.bfloat16)
    cap = _Capture()
    core.diagnostic_callback = cap
    repaired, info = core.repair(base, q, k, v, route)
    torch.cuda.synchronize()
    assert info["repair_feature_dim"] == D + role_dim and info["repair_rank"] == rank
    rows = cap.get("probe_rows").cpu().numpy()
    w = cap.get("probe_weights").cpu().numpy()
    xfit = cap.get("fit_features").cpu().numpy()
    yfit = cap.get("fit_targets").cpu().numpy()
    dense = cap.get("dense_probe").cpu().numpy()
    bn = base.reshape(H, N, D).float().cpu().numpy()
    role = route.q_role_features.cpu().numpy()
    want_x = np.take_along_axis(bn, rows[..., None].astype(np.int64), 1)
    if role_dim:
        want_x = np.concatenate((want_x, np.take_along_axis(role, rows[..., None].astype(np.int64), 1)), axis=2)
    assert np.array_equal(xfit, want_x) and np.array_equal(yfit, dense - want_x[:, :, :D])
    state = oracle.fit_reduced_rank_residual(xfit, yfit, cfg.repair_rank, cfg.repair_ridge, w,
                                             basis_source=cfg.repair_basis_source, output_basis_backend="skinny",
                                             decomposition_backend="triton_top16" if rank == 16 else "eigh")
    ref = oracle.repair_apply(bn, *state, cfg.repair_alpha, cfg.repair_norm_cap, role=role if role_dim else None)
    for h in range(H):
        ref[h, rows[h]] = dense[h]
    got = repaired.reshape(H, N, D).float().cpu().numpy()
    err = np.abs(got - ref)
    assert (err <= 1e-2 + 2.0 ** -8 * np.abs(ref)).all(), float(err.max())


def test_n8_route_top_p_budgets_and_attention_mass(dev, oracle):
    """selector_budget_mode svg_ear_top_p: budgets from the fp32 top-p rule on the new Q and
    K centroids, clamped, and the pair density they imply; selector_policy attention_mass."""
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    q, k, v = _inputs(dev, seed=9)
    B, H, N, D = q.shape
    cfg = N8V6Config(num_q_centroids=48, num_k_centroids=160, kmeans_iter_init=4, probe_rows=16,
                     selector_budget_mode="svg_ear_top_p", svg_ear_top_p=0.8, adaptive_budget_min_density=0.02,
                     adaptive_budget_max_density=0.5, selector_policy="attention_mass")
    core = N8V6Core(cfg)
    cap = _Capture()
    core.diagnostic_callback = cap
    route = core.route(q, k, v)
    torch.cuda.synchronize()
    ksz = route.k_cluster_sizes.cpu().numpy()
    qsz = route.q_cluster_sizes.cpu().numpy()
    want = oracle.svg_top_p_key_budgets(core.q_centroids.cpu().numpy(), core.k_centroids.cpu().numpy(), ksz, 0.8)
    want = np.clip(want, math.ceil(0.02 * N), math.floor(0.5 * N))
    budgets = cap.get("requested_key_budget").cpu().numpy()
    assert (budgets == want).all()
    dens = ((want * qsz).sum(1) / float(N * N)).mean()
    assert abs(route.base_video_density - dens) <= 1e-6
    scores = cap.get("svg_ear_scores").cpu().numpy()
    ks_np = route.k_permuted.reshape(H, -1, D).float().cpu().numpy()
    ref = oracle.attention_mass_scores(core.q_centroids.cpu().numpy(), ks_np, ksz, 1)
    _check_scores(scores, ref)
    assert (route.video_dynamic_map.cpu().numpy() == oracle.select_budget(scores, ksz, budgets, 1)[:, 1:, 1:]).all()


def test_n8_hunyuan_composition_default_config(dev, oracle):
    """The HunyuanVideo adapter's N8 step (hunyuanvideo.py:160-239) at the default N8V6Config
    (300 Q / 1000 K clusters, ranks 64 / 48, 64 probes, fixed density 0.22): video tokens plus
    a 256-token text suffix of which 77 are the prompt; route with the full K/V layout, the
    padded block map, block-sparse attention, inverse permutation, repair.  The base output
    against the float64 masked attention (192 sampled rows), the repaired video against the
    oracle's repair of the GPU base, the text rows against dense attention."""
    import torch.nn.functional as F

    from sparsepr_amd.kernels.permute import apply_inverse_permutation_triton, permute_tensor_by_labels_triton
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    qv, kv, vv = _inputs(dev, heads=2, frames=3, h=48, w=64, seed=11)  # 9,216 video tokens
    B, H, Nv, D = qv.shape
    text, prompt = 256, 77
    g = torch.Generator(device=dev).manual_seed(5)
    extra = [(0.8 * torch.randn((B, H, text, D), device=dev, generator=g)).to(torch.bfloat16) for _ in range(3)]
    query, key, value = (torch.cat((a, b), dim=2) for a, b in zip((qv, kv, vv), extra))
    cfg = N8V6Config()
    core = N8V6Core(cfg)
    route = core.route(qv, kv, vv, always_attended_keys=prompt, total_key_tokens=Nv + prompt, k_full_source=key,
                       v_full_source=value)
    assert route.permuted_includes_suffix and route.k_permuted.shape == key.shape
    # the adapter's query order and padded map (hunyuanvideo.py:189-222)
    q_order = torch.argsort(route.q_labels, dim=-1, stable=True).to(torch.int32).contiguous()
    q_full = torch.cat((q_order, torch.arange(Nv, Nv + text, device=dev, dtype=torch.int32).expand(B * H, -1)), 1)
    q_perm, _ = permute_tensor_by_labels_triton(query, None, dim=2, sorted_indices=q_full.contiguous())
    qc, kc = route.video_dynamic_map.shape[-2:]
    block_map = F.pad(route.video_dynamic_map.view(B, H, qc, kc), (0, 2, 0, 2), value=False)
    block_map[:, :, :-1, -2] = True
    block_map[:, :, -2, :-1] = True
    block_map[:, :, -1, -1] = True
    qs = F.pad(route.q_cluster_sizes.view(B, H, qc), (0, 2), value=0)
    ks = F.pad(route.k_cluster_sizes.view(B, H, kc), (0, 2), value=0)
    qs[:, :, -2:] = torch.tensor([prompt, text - prompt], device=dev, dtype=qs.dtype)
    ks[:, :, -2:] = torch.tensor([prompt, text - prompt], device=dev, dtype=ks.dtype)
    out_perm = dynamic_block_sparse_fwd_flashinfer(q_perm, route.k_permuted, route.v_permuted, block_map, qs, ks,
                                                   is_cpu=False)
    base_video = apply_inverse_permutation_triton(out_perm[:, :, :Nv], q_order, dim=2)
    repaired, info = core.repair(base_video, qv, key[:, :, :Nv + prompt], value[:, :, :Nv + prompt], route)
    torch.cuda.synchronize()
    assert 0.0 < float(info["effective_video_density"]) <= 1.0
    # float64 reference of the base on sampled rows: a video query in q-cluster a sees the
    # video keys of its kept k-clusters plus the prompt keys
    rng = np.random.default_rng(3)
    vmap = route.video_dynamic_map.cpu().numpy()
    ql = route.q_labels.cpu().numpy()
    kl = route.k_labels.cpu().numpy()
    for h in range(H):
        qh = qv[0, h].float().cpu().numpy()
        kh = key[0, h, :Nv + prompt].float().cpu().numpy()
        vh = value[0, h, :Nv + prompt].float().cpu().numpy()
        rows = np.sort(rng.choice(Nv, 96, replace=False))
        mask = np.concatenate((vmap[h][ql[h, rows]][:, kl[h]], np.ones((rows.size, prompt), bool)), 1)
        s = np.where(mask, qh[rows].astype(np.float64) @ kh.T.astype(np.float64) / math.sqrt(D), -np.inf)
        e = np.exp(s - s.max(1, keepdims=True))
        ref = (e @ vh.astype(np.float64)) / e.sum(1, keepdims=True)
        got = base_video[0, h, rows].float().cpu().numpy()
        assert np.abs(got - ref).max() <= 2e-2
        # probes from the role features, exact; then the repair of the GPU base by the oracle
        rr = route.probe_rows[h].cpu().numpy()
        rw = route.probe_weights[h].cpu().numpy()
        feats = route.q_role_features[h:h + 1].cpu().numpy()
        er, ew = oracle.select_role_equal_probes_vectorized(feats, ql[h:h + 1], cfg.num_q_centroids, cfg.probe_rows)
        assert (rr == er[0]).all() and np.allclose(rw, ew[0], rtol=1e-6)
        bh_np = base_video[0, h].float().cpu().numpy()
        gr = repaired[0, h].float().cpu().numpy()
        # the probe rows of the output are the GPU's dense probe attention (bf16 operands and
        # probabilities): within the attention bound of the float64 attention
        dense_ref = oracle.dense_attention(qh[rr][None], kh[None], vh[None])[0]
        dense = gr[rr][None]
        assert np.abs(dense[0] - dense_ref).max() <= 2e-2
        # the repair of the GPU base fitted to those probes by the float64 oracle on the
        # reference GPU's route (64 probes < D: the "skinny" top-16 subspace basis,
        # n8_v6.py:1310-1320); both fits see the same targets
        xfit = bh_np[rr][None]
        state = oracle.fit_reduced_rank_residual(xfit, dense - xfit, cfg.repair_rank, cfg.repair_ridge, rw[None],
                                                 output_basis_backend="skinny", decomposition_backend="triton_top16")
        ref_out = oracle.repair_apply(bh_np[None], *state, cfg.repair_alpha, 0.0)[0]
        ref_out[rr] = dense[0]
        # how far the exact eigenbasis (the reference's CPU route) would put the output
        exact = oracle.fit_reduced_rank_residual(xfit, dense - xfit, cfg.repair_rank, cfg.repair_ridge, rw[None])
        exact_out = oracle.repair_apply(bh_np[None], *exact, cfg.repair_alpha, 0.0)[0]
        exact_out[rr] = dense[0]
        ce, ct = exact_out - bh_np, ref_out - bh_np
        cos = (ce * ct).sum(1) / np.maximum(np.linalg.norm(ce, axis=1) * np.linalg.norm(ct, axis=1), 1e-30)
        print(f"head {h}: top-16 vs exact basis: output max-abs {np.abs(exact_out - ref_out).max():.4g}, "
              f"correction max-abs {np.abs(ct).max():.4g}, min row cosine of the corrections {cos.min():.4f}")
        # bf16 output: one ulp of the value (a rounding flip between the fp32 and float64
        # corrections) plus 1e-2 for the fp32 fit
        err = np.abs(gr - ref_out)
        bound = 1e-2 + 2.0 ** -8 * np.abs(ref_out)
        worst = np.unravel_index(np.argmax(err - bound), err.shape)
        assert (err <= bound).all(), (h, worst, float(err[worst]), float(ref_out[worst]), float(err.max()))
    # text rows (hunyuanvideo.py:203-207): the prompt queries see every video key and the
    # prompt keys; the padding queries see only the padding keys
    tq = query[0, :, Nv:].float().cpu().numpy()
    full_k = key[0].float().cpu().numpy()
    full_v = value[0].float().cpu().numpy()
    for h in range(H):
        seen = oracle.dense_attention(tq[h][None, :prompt], full_k[h][None, :Nv + prompt],
                                      full_v[h][None, :Nv + prompt])[0]
        assert np.abs(out_perm[0, h, Nv:Nv + prompt].float().cpu().numpy() - seen).max() <= 2e-2
        pad = oracle.dense_attention(tq[h][None, prompt:], full_k[h][None, Nv + prompt:], full_v[h][None, Nv + prompt:])[0]
        assert np.abs(out_perm[0, h, Nv + prompt:].float().cpu().numpy() - pad).max() <= 2e-2
