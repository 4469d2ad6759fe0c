"""N8-V6 method core: route carrier types and the current-step probe repair
(drop-in for src/sparsepr/models/common/n8_v6.py on the sparse-attention path).

`N8V6Core.repair` runs entirely on the HIP kernels (probe selection, dense probe
attention, fit preparation, apply, exact scatter) plus the small fp32 RRR fit
on the GPU.  The N8 role-space router (`route`) is not part of this library:
its SVG-EAR selector scores and role projections are (sparsepr_amd.kernels.svg_ear,
sparsepr_amd.kernels.role_projection), its role-metric factors and orchestration
are not.  The top-p router of `sparsepr_amd.layer` produces an `N8V6Route` that
`repair` consumes.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels.attention import dense_attention
from .kernels.residual_repair import n8_exact_probe_scatter_triton, n8_prepare_output_repair_fit_triton
from .residual_repair import (
    MODE_FIRST_TOKEN,
    MODE_ROUNDS,
    MODE_VECTORIZED,
    apply_reduced_rank_residual,
    fit_reduced_rank_residual,
    recover_nonfinite_rrr_state,
    select_probes,
)


def _effective_density(base_density, count: int, tokens: int):
    """min(1, base + M / N); a device-tensor density stays on the device (no sync)."""
    if torch.is_tensor(base_density):
        return (base_density + count / float(tokens)).clamp(max=1.0)
    return min(1.0, base_density + count / float(tokens))


@dataclass(frozen=True)
class N8V6Config:
    """Immutable N8-V6 configuration (field names and defaults of n8_v6.py:233-349)."""

    num_q_centroids: int = 300
    num_k_centroids: int = 1000
    target_density: float = 0.22
    role_q_rank: int = 64
    role_k_rank: int = 48
    role_v_rank: int = 16
    role_v_weight: float = 0.0
    metric_sample_tokens: int = 2048
    kmeans_iter_init: int = 25
    kmeans_iter_step: int = 2
    kmeans_backend: str = "flash"
    factor_power_iters: int = 2
    factor_orthogonalization: str = "each_cholesky_qr2"
    factor_ritz_mode: str = "rayleigh_cholesky"
    factor_rayleigh_ridge: float = 1e-4
    factor_cholesky_qr_ridge: float = 1e-5
    factor_refresh_every: int = 1
    probe_rows: int = 64
    repair_rank: int = 16
    repair_ridge: float = 0.1
    repair_alpha: float = 1.0
    repair_norm_cap: float = 0.0
    repair_features: str = "output"
    repair_basis_source: str = "raw_residual"
    probe_selection_policy: str = "role_equal_centroid"
    selector_block_q: int = 32
    selector_block_n: int = 16
    selector_num_warps: int = 2
    selector_policy: str = "svg_ear_value"
    selector_budget_mode: str = "fixed_density"
    svg_ear_top_p: float = 0.85
    adaptive_budget_min_density: float = 0.0
    adaptive_budget_max_density: float = 1.0
    grouped_svg_ear_router: bool = False
    role_projection_block_m: int = 32
    role_projection_num_warps: int = 2
    repair_block_n: int = 16
    repair_num_warps: int = 2
    repair_num_stages: int = 1
    repair_input_precision: str = "tf32"
    compile_role_kv_projection: bool = True
    role_kv_matmul_precision: str = "high"
    profile_breakdown: bool = False

    def validate(self, head_dim: int | None = None) -> None:
        if not 0.0 < self.target_density <= 1.0:
            raise ValueError(f"target_density must be in (0,1], got {self.target_density}.")
        if self.probe_rows <= 0 or self.repair_rank <= 0:
            raise ValueError("N8 probe_rows and repair_rank must be positive.")
        if self.factor_refresh_every <= 0:
            raise ValueError("factor_refresh_every must be positive.")
        if self.role_kv_matmul_precision not in {"highest", "high", "medium"}:
            raise ValueError(f"role_kv_matmul_precision must be highest, high, or medium; got "
                             f"{self.role_kv_matmul_precision!r}.")
        if self.probe_rows > self.num_q_centroids:
            raise ValueError("Vectorized role-equal probes require M <= Q clusters.")
        if self.role_v_weight < 0.0:
            raise ValueError("role_v_weight must be non-negative.")
        if self.repair_norm_cap < 0.0:
            raise ValueError("repair_norm_cap must be non-negative.")
        if self.repair_features not in {"output", "output_role"}:
            raise ValueError(f"repair_features must be output or output_role; got {self.repair_features!r}.")
        if self.repair_features == "output_role":
            # residual_repair.py:388-475,737-797 (role features appended to the fit's
            # features) has no HIP kernels here; refuse it instead of running the
            # output-only repair under the other name.
            raise NotImplementedError(
                "repair_features='output_role' is not supported by the MI355X build: the role-feature fit "
                "preparation and apply kernels are not built; use repair_features='output'.")
        if self.repair_basis_source not in {"raw_residual", "fitted_residual"}:
            raise ValueError(f"repair_basis_source must be raw_residual or fitted_residual; got "
                             f"{self.repair_basis_source!r}.")
        if self.selector_policy not in {"svg_ear_value", "attention_mass"}:
            raise ValueError(f"selector_policy must be svg_ear_value or attention_mass; got "
                             f"{self.selector_policy!r}.")
        if self.selector_budget_mode not in {"fixed_density", "svg_ear_top_p"}:
            raise ValueError(f"selector_budget_mode must be fixed_density or svg_ear_top_p; got "
                             f"{self.selector_budget_mode!r}.")
        if not 0.0 < self.svg_ear_top_p <= 1.0:
            raise ValueError(f"svg_ear_top_p must be in (0,1], got {self.svg_ear_top_p}.")
        if not 0.0 <= self.adaptive_budget_min_density <= self.adaptive_budget_max_density <= 1.0:
            raise ValueError("Adaptive budget densities must satisfy 0 <= minimum <= maximum <= 1.")
        if self.probe_selection_policy not in {"role_equal_centroid", "first_token_largest_groups"}:
            raise ValueError(f"probe_selection_policy must be role_equal_centroid or first_token_largest_groups; "
                             f"got {self.probe_selection_policy!r}.")
        if head_dim is not None and max(self.role_q_rank, self.role_k_rank, self.role_v_rank) > head_dim:
            raise ValueError(f"N8 role rank exceeds head dimension {head_dim}.")


@dataclass
class N8V6Route:
    """Routing result consumed by the attention call and by `N8V6Core.repair`
    (fields of n8_v6.py:351-369, plus the optional q-group centers that let
    repair skip recomputing them)."""

    q_labels: torch.Tensor
    k_labels: torch.Tensor
    q_cluster_sizes: torch.Tensor
    k_cluster_sizes: torch.Tensor
    video_dynamic_map: torch.Tensor
    q_role_features: torch.Tensor
    k_permuted: torch.Tensor | None  # None when the consumer gathers through k_sorted_indices
    v_permuted: torch.Tensor | None
    k_sorted_indices: torch.Tensor
    base_video_density: float
    q_kmeans_iters: int
    k_kmeans_iters: int
    permuted_includes_suffix: bool = False
    probe_rows: torch.Tensor | None = None
    probe_weights: torch.Tensor | None = None
    q_role_centers: torch.Tensor | None = None


class N8V6Core:
    """Per-attention-layer N8-V6 state: the last finite repair state (carried
    across denoising steps for non-finite recovery) and the fit buffers."""

    def __init__(self, config: N8V6Config, *, validate: bool = True):
        if validate:
            config.validate()
        self.config = config
        self.repair_state_current = None
        self.repair_recovery_mask = None
        self.route_call_index = 0
        self._fit_feature_buffer = None
        self._dense_probe_buffer = None
        self._fit_target_buffer = None
        self.last_repair_profile: dict = {}

    def reset(self) -> None:
        self.__init__(self.config, validate=False)

    def route(self, *args, **kwargs):
        raise NotImplementedError(
            "The N8 role-space router is not provided by sparsepr_amd: its metric covariance/factor "
            "step and route orchestration are not built (its SVG-EAR scores and role projections are: "
            "sparsepr_amd.kernels.svg_ear, sparsepr_amd.kernels.role_projection); use "
            "sparsepr_amd.layer.SparsePRAttention.route (top-p cluster routing)."
        )

    def repair(self, base_video, q_video, k_full, v_full, route: N8V6Route):
        """Current-step M-probe / rank-r repair of video rows (reference n8_v6.py:1174-1444).

        base_video, q_video [B, H, N, D]; k_full, v_full [B, H, N', D] bf16.
        Returns (corrected [B, H, N, D], info dict)."""
        batch, heads, tokens, dim = base_video.shape
        bh = batch * heads
        cfg = self.config
        if cfg.repair_features != "output":
            raise NotImplementedError(f"repair_features={cfg.repair_features!r} is not supported by the MI355X "
                                      "build; only the output-feature repair is built.")
        base = base_video.contiguous().view(bh, tokens, dim)
        if route.probe_rows is not None and route.probe_weights is not None:
            rows, weights = route.probe_rows, route.probe_weights
            cache_hit = True
        else:
            cache_hit = False
            feats = route.q_role_features
            count = min(cfg.probe_rows, tokens)
            if cfg.probe_selection_policy == "first_token_largest_groups":
                mode = MODE_FIRST_TOKEN
            else:
                mode = MODE_VECTORIZED if count <= cfg.num_q_centroids else MODE_ROUNDS
            sizes = route.q_cluster_sizes.reshape(bh, -1).to(torch.int32) if route.q_cluster_sizes is not None else None
            rows, weights = select_probes(feats, route.q_labels.reshape(bh, tokens), cfg.num_q_centroids,
                                          cfg.probe_rows, mode, centers=route.q_role_centers, sizes=sizes)
            route.probe_rows = rows
            route.probe_weights = weights
        count = int(rows.shape[1])
        q_flat = q_video.contiguous().view(bh, tokens, dim)
        from .flash_kmeans.kmeans_impl import gather_rows

        q_probe = gather_rows(q_flat, rows)
        kf = k_full.reshape(bh, -1, dim)
        vf = v_full.reshape(bh, -1, dim)
        dense_probe = dense_attention(q_probe, kf, vf, out_dtype=q_video.dtype if q_video.dtype == torch.bfloat16
                                      else torch.float32)
        shape = (bh, count, dim)
        if self._fit_feature_buffer is None or tuple(self._fit_feature_buffer.shape) != shape:
            self._fit_feature_buffer = torch.empty(shape, device=base.device, dtype=torch.float32)
            self._dense_probe_buffer = torch.empty(shape, device=base.device, dtype=torch.float32)
            self._fit_target_buffer = torch.empty(shape, device=base.device, dtype=torch.float32)
        x_fit, dense_probe_f, y_fit = n8_prepare_output_repair_fit_triton(
            base, dense_probe, rows, self._fit_feature_buffer, self._dense_probe_buffer, self._fit_target_buffer)
        state = fit_reduced_rank_residual(
            x_fit, y_fit, rank=min(cfg.repair_rank, count, dim), ridge=cfg.repair_ridge, weights=weights,
            output_basis_backend="skinny", cache_identity=True, fit_backend="dual_cholesky",
            decomposition_backend="eigh", basis_source=cfg.repair_basis_source)
        state, self.repair_recovery_mask, policy = recover_nonfinite_rrr_state(state, self.repair_state_current)
        self.repair_state_current = state
        x_mean, x_scale, y_mean, left, basis = state
        corrected = apply_reduced_rank_residual(base, None, x_mean, x_scale, y_mean, left, basis, cfg.repair_alpha,
                                                cfg.repair_norm_cap)
        n8_exact_probe_scatter_triton(corrected, rows, dense_probe_f)
        info = {
            "probe_rows": count,
            "probe_selection_policy": cfg.probe_selection_policy,
            "probe_selection_cache_hit": cache_hit,
            "repair_rank": min(cfg.repair_rank, count, dim),
            "repair_feature_dim": dim,
            "repair_features": cfg.repair_features,
            "repair_basis_source": cfg.repair_basis_source,
            "repair_backend": "hip_mi355x",
            "repair_recovery_policy": policy,
            "effective_video_density": _effective_density(route.base_video_density, count, tokens),
        }
        return corrected.view_as(base_video), info
