"""N8-V6 method core: role routing and the current-step probe repair (drop-in for
src/sparsepr/models/common/n8_v6.py on the sparse-attention path).

`N8V6Core.route` computes the video-token cluster map: role metrics and factors (cold
eigen factor, then warm subspace updates), TF32 role projections, role-space k-means of K
and Q, original-space centroids, the K/V permutation, SVG-EAR / attention-mass selector
scores, fixed-density or top-p key budgets and the exact budget selector.
`N8V6Core.repair` runs the probe selection, dense probe attention, fit preparation, the
reduced-rank fit, the apply and the exact scatter.  Every compute step is a HIP kernel of
libsparsepr_hip.so.  Configurations outside the kernels' sizes (head dims other than 64 and
128, role ranks above 64, more than 128 K role features, output_role with a Q role rank that
is not a multiple of 16) raise NotImplementedError.
"""

from __future__ import annotations

import math
import os
import time
from dataclasses import dataclass

import torch

from . import _lib, kmeans_utils
from . import operator_kmeans as _ok
from .kernels import role_metric as _rm
from .kernels.attention import dense_attention
from .kernels.permute import argsort_labels, permute_tensor_by_labels_triton
from .kernels.role_projection import (role_k_projection_normalize, role_kv_projection_normalize,
                                      role_projection_rms_triton)
from .kernels.selection import MODE_N8_NATIVE, MODE_TRITON, select_budget, top_p_key_budgets
from .kernels.svg_ear import (attention_mass_scores_triton, svg_ear_grouped_value_error_scores_triton,
                              svg_ear_value_error_scores_triton)
from .kernels.residual_repair import (n8_exact_probe_scatter_triton, n8_prepare_output_repair_fit_triton,
                                      n8_prepare_repair_fit_triton)
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
        if self.repair_features == "output_role" and (self.role_q_rank % 16 != 0 or self.role_q_rank > 64):
            # the role-feature apply kernel takes 16, 32, 48 or 64 role features per row
            raise NotImplementedError(
                f"repair_features='output_role' on the MI355X kernels needs role_q_rank in (16, 32, 48, 64); got "
                f"{self.role_q_rank}.")
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


_ENV_OFF = {"", "0", "false", "no", "off"}


def _env_flag(name: str) -> bool:
    return os.environ.get(name, "0").lower() not in _ENV_OFF


class N8V6Core:
    """Per-attention-layer N8-V6 state (n8_v6.py:371-406): role factors and their subspace
    states, the previous centroids (warm starts and empty-cluster fallbacks), the last finite
    repair state, and the fit buffers.  Single-threaded and stream ordered."""

    def __init__(self, config: N8V6Config, *, validate: bool = True):
        if validate:
            config.validate()
        self.config = config
        self.q_centroids = None
        self.k_centroids = None
        self.v_centroids = None
        self.q_factor_state = None
        self.k_factor_state = None
        self.v_factor_state = None
        self.q_factor_current = None
        self.k_factor_current = None
        self.v_factor_current = None
        self.q_factor_recovery_mask = None
        self.k_factor_recovery_mask = None
        self.v_factor_recovery_mask = None
        self.repair_state_current = None
        self.repair_recovery_mask = None
        self.route_call_index = 0
        self._fit_feature_buffer = None
        self._dense_probe_buffer = None
        self._fit_target_buffer = None
        self._full_k_order = None
        self.last_route_profile: dict = {}
        self.last_repair_profile: dict = {}
        self.diagnostic_callback = None

    @property
    def initialized(self) -> bool:
        return self.q_centroids is not None

    def reset(self) -> None:
        self.__init__(self.config, validate=False)

    def _emit_diagnostic(self, stage: str, *, tensors: dict, scalars: dict) -> None:
        callback = self.diagnostic_callback
        if callback is not None:
            callback(stage, tensors, {"core_route_call": int(self.route_call_index), **scalars})

    def _full_key_order(self, video_order: torch.Tensor, video_tokens: int, total_tokens: int) -> torch.Tensor:
        """The video key order followed by the identity over the suffix (n8_v6.py:407-432)."""
        bh = int(video_order.shape[0])
        expected = (bh, total_tokens)
        if (self._full_k_order is None or tuple(self._full_k_order.shape) != expected
                or self._full_k_order.device != video_order.device):
            self._full_k_order = torch.empty(expected, device=video_order.device, dtype=torch.int32)
            suffix = torch.arange(video_tokens, total_tokens, device=video_order.device, dtype=torch.int32)
            self._full_k_order[:, video_tokens:].copy_(suffix.unsqueeze(0))
        self._full_k_order[:, :video_tokens].copy_(video_order)
        return self._full_k_order

    def _check_route_config(self, dim: int) -> None:
        cfg = self.config
        # the names warm_subspace_metric_factor accepts (operator_kmeans.py:308-326)
        if cfg.factor_orthogonalization not in _rm.ORTHO:
            raise RuntimeError(f"Unknown subspace orthogonalization {cfg.factor_orthogonalization!r}.")
        if cfg.factor_ritz_mode not in _rm.RITZ:
            raise RuntimeError(f"Unknown Rayleigh--Ritz mode {cfg.factor_ritz_mode!r}.")
        ranks = (cfg.role_q_rank, cfg.role_k_rank) + ((cfg.role_v_rank,) if cfg.role_v_weight > 0.0 else ())
        k_feature_dim = cfg.role_k_rank + (cfg.role_v_rank if cfg.role_v_weight > 0.0 else 0)
        # the role-space k-means takes feature dims that are multiples of 16 up to 128
        if (max(ranks) > 64 or dim not in (64, 128) or k_feature_dim > 128 or k_feature_dim % 16
                or cfg.role_q_rank % 16):
            raise NotImplementedError("N8 routing on the MI355X kernels needs head_dim 64 or 128, ranks <= 64, a "
                                      "Q role rank that is a multiple of 16 and K role features (role_k_rank, "
                                      "+ role_v_rank when role_v_weight > 0) a multiple of 16 up to 128.")

    def _kv_precision(self) -> str:
        """The fp32 matmul precision of the K (and V) role projections (n8_v6.py:658-704): the
        compiled projections run under role_kv_matmul_precision; the uncompiled ones are plain
        fp32 bmm (project_tokens), which is "highest"."""
        cfg = self.config
        return cfg.role_kv_matmul_precision if cfg.compile_role_kv_projection else "highest"

    def _updated_factor(self, metric, previous, current, rank):
        """n8_v6.py:478-519: the cold eigen factor on the first call, then one warm subspace
        update per call with per-head reuse of the previous factor when it fails."""
        cfg = self.config
        if previous is None:
            factor = _ok.metric_factor(metric, rank)
            recovered = torch.zeros(metric.shape[0], device=metric.device, dtype=torch.bool)
            return factor, factor, recovered
        if current is None:
            raise RuntimeError("Warm role-factor state is missing its current factor.")
        return _rm.warm_metric_factor(
            metric, previous, rank, prev_factor=current, power_iters=cfg.factor_power_iters,
            orthogonalization=cfg.factor_orthogonalization, ritz_mode=cfg.factor_ritz_mode,
            rayleigh_ridge=cfg.factor_rayleigh_ridge, cholesky_qr_ridge=cfg.factor_cholesky_qr_ridge)

    def route(self, q_video, k_video, v_video, *, gqa_group_size: int = 1, always_attended_keys: int = 0,
              total_key_tokens: int | None = None, k_full_source=None, v_full_source=None) -> N8V6Route:
        """The N8-V6 video-token map (n8_v6.py:521-1172): role metrics and factors, role-space
        k-means of K then Q, original-space centroids, the K/V permutation, the selector
        scores, the budgets and the exact budget selector, all on the HIP kernels."""
        if q_video.shape != k_video.shape or q_video.shape != v_video.shape or q_video.ndim != 4:
            raise RuntimeError(
                "N8-V6 expects matching [B,H,N,D] video Q/K/V; got "
                f"Q={tuple(q_video.shape)}, K={tuple(k_video.shape)}, V={tuple(v_video.shape)}."
            )
        batch, heads, tokens, dim = q_video.shape
        self.config.validate(dim)
        self._check_route_config(dim)
        _lib.require_gpu(q_video, k_video, v_video, what="N8V6Core.route")
        bh = batch * heads
        cfg = self.config
        q = q_video.contiguous().view(bh, tokens, dim)
        profile_breakdown = bool(cfg.profile_breakdown or getattr(self, "profile_breakdown_active", False))
        group = int(gqa_group_size)
        if group <= 0 or heads % group != 0:
            raise ValueError(f"gqa_group_size must divide the query-head count; got H={heads}, G={group}.")
        kv_heads = heads // group
        if group > 1:
            k = k_video[:, ::group].contiguous().view(batch * kv_heads, tokens, dim)
            v = v_video[:, ::group].contiguous().view(batch * kv_heads, tokens, dim)
            _, q_metric_source = _ok.gqa_metric_sources(q_video, k_video, q_cluster_heads=heads,
                                                        k_cluster_heads=kv_heads, gqa_group_size=group)
            metric_sample_tokens = cfg.metric_sample_tokens * group
        else:
            k = k_video.contiguous().view(bh, tokens, dim)
            v = v_video.contiguous().view(bh, tokens, dim)
            q_metric_source = q
            metric_sample_tokens = cfg.metric_sample_tokens
        self.last_route_profile = {
            "n8_profile_enabled": profile_breakdown, "n8_gqa_key_sharing": bool(group > 1),
            "n8_gqa_group_size": group, "n8_q_cluster_heads": heads, "n8_k_cluster_heads": kv_heads,
            "n8_k_runtime_heads": heads, "n8_selector_budget_mode": cfg.selector_budget_mode,
            "n8_svg_ear_top_p": float(cfg.svg_ear_top_p),
            "n8_adaptive_budget_min_density": float(cfg.adaptive_budget_min_density),
            "n8_adaptive_budget_max_density": float(cfg.adaptive_budget_max_density),
            "n8_backend": "hip_mi355x",
        }
        started = [time.perf_counter()]

        def profile_mark(name: str) -> None:
            if not profile_breakdown:
                return
            torch.cuda.synchronize(q_video.device)
            now = time.perf_counter()
            self.last_route_profile[f"n8_route_{name}_ms"] = (now - started[0]) * 1000.0
            started[0] = now

        if profile_breakdown:
            torch.cuda.synchronize(q_video.device)
            started[0] = time.perf_counter()

        # ---- K (and V) role factors (n8_v6.py:611-657)
        joint_v = cfg.role_v_weight > 0.0
        refresh = (self.q_factor_current is None or self.k_factor_current is None
                   or (joint_v and self.v_factor_current is None)
                   or self.route_call_index % cfg.factor_refresh_every == 0)
        if refresh:
            k_metric = _ok.key_metric_from_queries(q_metric_source, metric_sample_tokens)
            v_metric = _ok.value_metric_from_values(v, cfg.metric_sample_tokens) if joint_v else None
            if self.diagnostic_callback is not None:
                metric_tensors = {"k_role_metric": k_metric}
                if v_metric is not None:
                    metric_tensors["v_role_metric"] = v_metric
                self._emit_diagnostic("clustering", tensors=metric_tensors,
                                      scalars={"phase": "kv_metrics_before_factorization"})
            k_factor, self.k_factor_state, self.k_factor_recovery_mask = self._updated_factor(
                k_metric, self.k_factor_state, self.k_factor_current, cfg.role_k_rank)
            self.k_factor_current = k_factor
            if v_metric is not None:
                v_factor, self.v_factor_state, self.v_factor_recovery_mask = self._updated_factor(
                    v_metric, self.v_factor_state, self.v_factor_current, cfg.role_v_rank)
                self.v_factor_current = v_factor
            else:
                v_factor = None
                self.v_factor_recovery_mask = torch.zeros(k_factor.shape[0], device=k_factor.device,
                                                          dtype=torch.bool)
        else:
            k_factor = self.k_factor_current
            v_factor = self.v_factor_current if joint_v else None
        profile_mark("kv_metric_factor")
        # ---- K role features and the warm start (n8_v6.py:658-704): the projection under the
        # K/V matmul precision, one RMS scale per head (and the weighted V features beside the K
        # ones when role_v_weight > 0)
        precision = self._kv_precision()
        if joint_v:
            k_features, k_scale, v_scale = role_kv_projection_normalize(k, v, k_factor, v_factor, cfg.role_v_weight,
                                                                        precision=precision)
        else:
            k_features, k_scale = role_k_projection_normalize(k, k_factor, precision=precision)
            v_scale = None
        k_init = None
        if self.k_centroids is not None:
            if joint_v:
                k_init = torch.empty((self.k_centroids.shape[0], self.k_centroids.shape[1], k_features.shape[2]),
                                     device=k_features.device, dtype=torch.float32)
                _rm.project_rows(self.k_centroids, k_factor, divisor=k_scale, precision=precision, out=k_init)
                _rm.project_rows(self.v_centroids, v_factor, divisor=v_scale, precision=precision,
                                 weight=cfg.role_v_weight, out=k_init, out_col=cfg.role_k_rank)
            else:
                k_init = _rm.project_rows(self.k_centroids, k_factor, divisor=k_scale, precision=precision)
        profile_mark("kv_projection_init")
        k_iters = cfg.kmeans_iter_step if self.initialized else cfg.kmeans_iter_init
        k_backend = cfg.kmeans_backend
        if k_backend == "n8_cuda_ext" and k_init is None:
            k_backend = "flash"
        k_res = kmeans_utils._lloyd_result(k_features, cfg.num_k_centroids, max_iters=k_iters,
                                           init_centroids=k_init, backend=k_backend)
        k_labels, k_sizes, k_iter = k_res.labels, k_res.sizes.long(), k_res.iters
        profile_mark("kmeans_k")
        # ---- original-space K and V centroids, one label traversal (n8_v6.py:719-726)
        self.k_centroids, self.v_centroids = _ok.joint_original_centroids(
            k, v, k_labels, k_sizes, x_empty_fallback=self.k_centroids, y_empty_fallback=self.v_centroids,
            sorted_labels=(k_res.sorted_idx, k_res.offsets))
        profile_mark("kv_centroids")
        # ---- Q role factor from the key centroids (n8_v6.py:728-755)
        if refresh:
            q_metric = _ok.query_metric_from_key_centroids(self.k_centroids, k_sizes)
            if self.diagnostic_callback is not None:
                self._emit_diagnostic("clustering", tensors={"q_role_metric": q_metric},
                                      scalars={"phase": "q_metric_before_factorization"})
            q_factor, self.q_factor_state, self.q_factor_recovery_mask = self._updated_factor(
                q_metric, self.q_factor_state, self.q_factor_current, cfg.role_q_rank)
            self.q_factor_current = q_factor
        else:
            q_factor = self.q_factor_current
        if group > 1:
            q_factor_runtime = q_factor.view(batch, kv_heads, dim, cfg.role_q_rank).repeat_interleave(
                group, dim=1).contiguous().view(bh, dim, cfg.role_q_rank)
        else:
            q_factor_runtime = q_factor
        profile_mark("q_metric_factor")
        # ---- Q role features, warm start, k-means, original-space Q centroids (n8_v6.py:756-804)
        q_features = role_projection_rms_triton(q, q_factor_runtime)
        q_init = None
        if self.q_centroids is not None:
            q_init = _rm.project_rows(self.q_centroids, q_factor_runtime, row_rms=True, eps=1e-6)
        profile_mark("q_projection_init")
        q_backend = cfg.kmeans_backend
        if q_backend == "n8_cuda_ext" and q_init is None:
            q_backend = "flash"
        q_res = kmeans_utils._lloyd_result(q_features, cfg.num_q_centroids, max_iters=k_iters,
                                           init_centroids=q_init, backend=q_backend)
        q_labels, q_sizes, q_iter = q_res.labels, q_res.sizes.long(), q_res.iters
        profile_mark("kmeans_q")
        self.q_centroids = _ok.original_centroids(q, q_labels, q_sizes, empty_fallback=self.q_centroids,
                                                  sorted_labels=(q_res.sorted_idx, q_res.offsets))
        profile_mark("q_centroids")
        # ---- GQA: K clusters shared by the query heads of a group (n8_v6.py:806-839)
        if group > 1:
            def per_q_head(t, *tail):
                return t.view(batch, kv_heads, *tail).repeat_interleave(group, dim=1).contiguous().view(
                    bh, *tail)

            k_labels_runtime = per_q_head(k_labels, tokens)
            k_sizes_runtime = per_q_head(k_sizes, cfg.num_k_centroids)
            k_centroids_runtime = per_q_head(self.k_centroids, cfg.num_k_centroids, dim)
            v_centroids_runtime = per_q_head(self.v_centroids, cfg.num_k_centroids, dim)
            k_order = argsort_labels(k_labels_runtime, cfg.num_k_centroids)[0]
        else:
            k_labels_runtime, k_sizes_runtime = k_labels, k_sizes
            k_centroids_runtime, v_centroids_runtime = self.k_centroids, self.v_centroids
            k_order = k_res.sorted_idx  # the stable argsort of the final labels
        if self.diagnostic_callback is not None:
            self._emit_diagnostic("clustering", tensors={
                "q_factor": q_factor, "k_factor": k_factor, "q_centroids": self.q_centroids,
                "k_centroids": self.k_centroids, "v_centroids": self.v_centroids, "q_cluster_sizes": q_sizes,
                "k_cluster_sizes": k_sizes, "q_factor_recovery_mask": self.q_factor_recovery_mask,
                "k_factor_recovery_mask": self.k_factor_recovery_mask},
                scalars={"phase": "cluster_result", "factor_refresh": bool(refresh), "q_kmeans_iters": int(q_iter),
                         "k_kmeans_iters": int(k_iter), "factor_recovery_policy": "reuse_previous_finite_factor"})
        # ---- K/V permuted once into cluster order (n8_v6.py:900-933)
        use_full_layout = k_full_source is not None or v_full_source is not None
        if use_full_layout:
            if k_full_source is None or v_full_source is None:
                raise ValueError("k_full_source and v_full_source must be provided together.")
            if k_full_source.shape != v_full_source.shape or k_full_source.ndim != 4:
                raise ValueError("Full K/V sources must have matching [B,H,N,D] shapes.")
            if tuple(k_full_source.shape[:2]) != (batch, heads) or k_full_source.shape[-1] != dim:
                raise ValueError("Full K/V sources do not match the video tensor head layout.")
            total_layout_tokens = int(k_full_source.shape[2])
            if total_layout_tokens < tokens:
                raise ValueError("Full K/V source is shorter than the video prefix.")
            full_order = self._full_key_order(k_order, tokens, total_layout_tokens)
            k_permuted, _ = permute_tensor_by_labels_triton(k_full_source, None, dim=2, sorted_indices=full_order)
            v_permuted, _ = permute_tensor_by_labels_triton(v_full_source, None, dim=2, sorted_indices=full_order)
            selector_k = k_permuted.reshape(bh, total_layout_tokens, dim)
            selector_v = v_permuted.reshape(bh, total_layout_tokens, dim)
        else:
            k_permuted, _ = permute_tensor_by_labels_triton(k_video, None, dim=2, sorted_indices=k_order)
            v_permuted, _ = permute_tensor_by_labels_triton(v_video, None, dim=2, sorted_indices=k_order)
            selector_k = k_permuted.reshape(bh, tokens, dim)
            selector_v = v_permuted.reshape(bh, tokens, dim)
        profile_mark("kv_permute")
        # ---- selector scores (n8_v6.py:934-990)
        use_grouped = bool(cfg.grouped_svg_ear_router and cfg.selector_policy == "svg_ear_value" and group > 1)
        if use_grouped:
            stored = int(selector_k.shape[1])
            k_native = selector_k.view(batch, heads, stored, dim)[:, ::group].contiguous().view(
                batch * kv_heads, stored, dim)
            v_native = selector_v.view(batch, heads, stored, dim)[:, ::group].contiguous().view(
                batch * kv_heads, stored, dim)
            scores = svg_ear_grouped_value_error_scores_triton(
                qcentroids=self.q_centroids, k_sorted=k_native, v_sorted=v_native, kcentroids=self.k_centroids,
                vcentroids=self.v_centroids, kcluster_sizes=k_sizes, gqa_group=group,
                block_q=min(cfg.selector_block_q, 16), block_n=cfg.selector_block_n,
                num_warps=max(4, cfg.selector_num_warps))
        elif cfg.selector_policy == "attention_mass":
            scores = attention_mass_scores_triton(
                qcentroids=self.q_centroids, k_sorted=selector_k, kcluster_sizes=k_sizes_runtime, gqa_group=1,
                block_q=cfg.selector_block_q, block_n=cfg.selector_block_n, num_warps=cfg.selector_num_warps,
                logical_tokens=tokens)
        else:
            scores = svg_ear_value_error_scores_triton(
                qcentroids=self.q_centroids, k_sorted=selector_k, v_sorted=selector_v,
                kcentroids=k_centroids_runtime, vcentroids=v_centroids_runtime, kcluster_sizes=k_sizes_runtime,
                gqa_group=1, var_k_diag=None, jensen_var_cap=0.0, block_q=cfg.selector_block_q,
                block_n=cfg.selector_block_n, num_warps=cfg.selector_num_warps, logical_tokens=tokens)
        profile_mark("selector_scores")
        if self.diagnostic_callback is not None:
            self._emit_diagnostic("svg_ear_selection", tensors={"svg_ear_scores": scores},
                                  scalars={"phase": "scores_before_budget_selection",
                                           "selector_policy": cfg.selector_policy,
                                           "grouped_svg_ear_router": use_grouped})
        # ---- key budgets (n8_v6.py:1004-1061)
        total_keys = int(total_key_tokens) if total_key_tokens is not None else tokens
        if total_keys < tokens or always_attended_keys < 0 or always_attended_keys > total_keys:
            raise ValueError(f"Invalid key accounting: video={tokens}, total={total_keys}, "
                             f"always={always_attended_keys}.")
        if cfg.selector_budget_mode == "fixed_density":
            base_total_density = max(0.0, cfg.target_density - cfg.probe_rows / float(tokens))
            target_keys = int(math.ceil(base_total_density * total_keys))
            budget = max(0, target_keys - int(always_attended_keys))
            budgets = torch.full((bh, cfg.num_q_centroids), budget, device=q_video.device, dtype=torch.int32)
            base_density = budget / float(tokens)
        else:
            budgets = top_p_key_budgets(self.q_centroids, k_centroids_runtime, k_sizes_runtime, cfg.svg_ear_top_p)
            budgets = budgets.clamp(min=int(math.ceil(cfg.adaptive_budget_min_density * tokens)),
                                    max=int(math.floor(cfg.adaptive_budget_max_density * tokens)))
            pair_density = (budgets * q_sizes).sum(dim=1).float() / float(tokens * tokens)
            base_density = float(pair_density.mean().item())
        # ---- exact budget selector (n8_v6.py:1062-1112): the n8_kernels semantics when
        # SPARSEPR_N8_CUDA_EXT_SELECTOR is set, else the Triton selector's
        mode = MODE_N8_NATIVE if _env_flag("SPARSEPR_N8_CUDA_EXT_SELECTOR") else MODE_TRITON
        routed = select_budget(scores, k_sizes_runtime, budgets, mode)
        video_map = routed[:, 1:, 1:]
        profile_mark("selector_budget")
        if self.diagnostic_callback is not None:
            self._emit_diagnostic("svg_ear_selection", tensors={"routed_map": routed, "requested_key_budget": budgets},
                                  scalars={"phase": "budget_selection_result",
                                           "selector_budget_mode": cfg.selector_budget_mode,
                                           "base_video_density": float(base_density)})
        result = N8V6Route(
            q_labels=q_labels, k_labels=k_labels_runtime, q_cluster_sizes=q_sizes, k_cluster_sizes=k_sizes_runtime,
            video_dynamic_map=video_map, q_role_features=q_features, k_permuted=k_permuted, v_permuted=v_permuted,
            k_sorted_indices=k_order, base_video_density=base_density, q_kmeans_iters=int(q_iter),
            k_kmeans_iters=int(k_iter), permuted_includes_suffix=use_full_layout)
        self.route_call_index += 1
        return result

    def repair(self, base_video, q_video, k_full, v_full, route: N8V6Route):
        """Current-step M-probe / rank-r repair of video rows (reference n8_v6.py:1174-1444).

        base_video, q_video [B, H, N, D]; k_full, v_full [B, H, N', D] bf16.
        Returns (corrected [B, H, N, D], info dict)."""
        return self.repair_finish(base_video, self.repair_probes(q_video, k_full, v_full, route), route)

    def repair_probes(self, q_video, k_full, v_full, route: N8V6Route):
        """The part of the repair that does not read the base output: probe rows and
        weights (cached on the route) and the dense attention of the probe queries over
        all keys.  It can run while the sparse attention computes the base."""
        batch, heads, tokens, dim = q_video.shape
        bh = batch * heads
        cfg = self.config
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
        q_flat = q_video.contiguous().view(bh, tokens, dim)
        from .flash_kmeans.kmeans_impl import gather_rows

        q_probe = gather_rows(q_flat, rows)
        kf = k_full.reshape(bh, -1, dim)
        vf = v_full.reshape(bh, -1, dim)
        dense_probe = dense_attention(q_probe, kf, vf, out_dtype=q_video.dtype if q_video.dtype == torch.bfloat16
                                      else torch.float32)
        return rows, weights, dense_probe, cache_hit

    def repair_finish(self, base_video, probes, route: N8V6Route):
        """The rest of the repair given repair_probes' result: fit on the probe rows of
        the base output, low-rank correction of every row, exact probe rows."""
        batch, heads, tokens, dim = base_video.shape
        bh = batch * heads
        cfg = self.config
        rows, weights, dense_probe, cache_hit = probes
        base = base_video.contiguous().view(bh, tokens, dim)
        count = int(rows.shape[1])
        # output_role: the Q role features join the fit's features (n8_v6.py:1246-1290)
        role = route.q_role_features.contiguous() if cfg.repair_features == "output_role" else None
        role_dim = 0 if role is None else int(role.shape[2])
        shape = (bh, count, dim + role_dim)
        if self._fit_feature_buffer is None or tuple(self._fit_feature_buffer.shape) != shape:
            self._fit_feature_buffer = torch.empty(shape, device=base.device, dtype=torch.float32)
            self._dense_probe_buffer = torch.empty((bh, count, dim), device=base.device, dtype=torch.float32)
            self._fit_target_buffer = torch.empty((bh, count, dim), device=base.device, dtype=torch.float32)
        if role is not None:
            x_fit, dense_probe_f, y_fit = n8_prepare_repair_fit_triton(
                base, role, dense_probe, rows, self._fit_feature_buffer, self._dense_probe_buffer,
                self._fit_target_buffer)
        else:
            x_fit, dense_probe_f, y_fit = n8_prepare_output_repair_fit_triton(
                base, dense_probe, rows, self._fit_feature_buffer, self._dense_probe_buffer, self._fit_target_buffer)
        if self.diagnostic_callback is not None:
            self._emit_diagnostic("probe_fit", tensors={"probe_rows": rows, "probe_weights": weights,
                                                        "dense_probe": dense_probe_f, "fit_features": x_fit,
                                                        "fit_targets": y_fit},
                                  scalars={"phase": "inputs_before_solver", "probe_count": count})
        # The reference's GPU route (n8_v6.py:1310-1320): with fewer probes than D the basis is
        # the top-16 subspace iteration, whose kernel takes exactly 64 probes at D = 128 (the
        # N8 default) and rank 16.  Other counts below D, which the reference's kernel refuses,
        # take the exact eigenbasis here.
        rank = min(cfg.repair_rank, count, dim)
        backend = "triton_top16" if (count, dim, rank) == (64, 128, 16) else "eigh"
        state = fit_reduced_rank_residual(
            x_fit, y_fit, rank=rank, ridge=cfg.repair_ridge, weights=weights,
            output_basis_backend="skinny", cache_identity=True, fit_backend="dual_cholesky",
            decomposition_backend=backend, basis_source=cfg.repair_basis_source)
        previous = self.repair_state_current
        state, self.repair_recovery_mask, policy = recover_nonfinite_rrr_state(state, previous)
        # The last finite state lives in buffers of its own, written in place, so that a
        # call captured in a HIP graph reads, on each replay, what the previous call wrote.
        if previous is not None and all(a.shape == b.shape and a.dtype == b.dtype for a, b in zip(previous, state)):
            for a, b in zip(previous, state):
                a.copy_(b)
            state = previous
        self.repair_state_current = state
        x_mean, x_scale, y_mean, left, basis = state
        corrected = apply_reduced_rank_residual(base, role, x_mean, x_scale, y_mean, left, basis, cfg.repair_alpha,
                                                cfg.repair_norm_cap)
        n8_exact_probe_scatter_triton(corrected, rows, dense_probe_f)
        info = {
            "probe_rows": count,
            "probe_selection_policy": cfg.probe_selection_policy,
            "probe_selection_cache_hit": cache_hit,
            "repair_rank": min(cfg.repair_rank, count, dim),
            "repair_feature_dim": dim + role_dim,
            "repair_features": cfg.repair_features,
            "repair_basis_source": cfg.repair_basis_source,
            "repair_backend": "hip_mi355x",
            "repair_recovery_policy": policy,
            "effective_video_density": _effective_density(route.base_video_density, count, tokens),
        }
        return corrected.view_as(base_video), info
