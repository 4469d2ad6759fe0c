"""One SparsePR attention layer on the MI355X kernels: the hot path end to end.

Composition (reference call sites):
  route   : flash k-means of Q and of K (Lloyd, fixed iterations), top-p
            cluster-pair map, K/V permutation  -- wan22.py:2221-2258 (SAP route),
            n8_v6.py:905-925 (K/V permute)
  attend  : block-sparse attention over the kept cluster pairs, reading Q and
            writing the output through the query sort index (the Q permutation
            and its inverse fused in)          -- hunyuanvideo.py:189-231
  repair  : N8 probe repair of the dropped blocks -- n8_v6.py:1174-1444
            (probes are role-equal representatives of the Q clusters; with the
            top-p route the role features are the queries themselves)

Every stage is a HIP kernel of libsparsepr_hip.so, the reduced-rank fit
included.  Nothing here synchronises the host.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .flash_kmeans.kmeans_impl import X_SQ_BF16, gather_rows, lloyd
from .kernels.attention import block_sparse_attention, plan_block_sparse
from .kernels.selection import density, topp_map
from .n8_v6 import N8V6Config, N8V6Core, N8V6Route
from .synthetic import first_k_indices


@dataclass(frozen=True)
class SparsePRConfig:
    num_q_centroids: int = 128
    num_k_centroids: int = 512
    kmeans_iters: int = 5
    top_p: float = 0.9
    min_kc_ratio: float = 0.0
    probe_rows: int = 128
    repair: bool = True
    repair_rank: int = 16
    repair_ridge: float = 0.1
    repair_alpha: float = 1.0
    repair_norm_cap: float = 0.0
    init_seed: int = 0
    x_sq_mode: int = X_SQ_BF16
    # Q's k-means and the repair's probe part (probe selection, dense probe attention)
    # run on a second stream beside K's k-means; results are the same either way.  None:
    # on when B*H*N is at least OVERLAP_MIN_TOKEN_HEADS (below that the layer is bound by
    # kernel launches, and the streams' events cost more than the overlap saves: 1.73 ms
    # against 1.45 ms at 2 heads x 4,096 tokens).
    overlap_streams: bool | None = None


OVERLAP_MIN_TOKEN_HEADS = 1 << 20


@dataclass
class LayerTimings:
    """Optional per-stage HIP events (recorded on the current stream)."""
    events: dict = field(default_factory=dict)

    def mark(self, name: str):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events[name] = ev

    def ms(self, a: str, b: str) -> float:
        return self.events[a].elapsed_time(self.events[b])


class SparsePRAttention:
    """Stateless across calls except the repair core's last finite RRR state."""

    def __init__(self, config: SparsePRConfig = SparsePRConfig()):
        self.config = config
        n8cfg = N8V6Config(num_q_centroids=config.num_q_centroids, num_k_centroids=config.num_k_centroids,
                           probe_rows=config.probe_rows, repair_rank=config.repair_rank,
                           repair_ridge=config.repair_ridge, repair_alpha=config.repair_alpha,
                           repair_norm_cap=config.repair_norm_cap)
        self.n8 = N8V6Core(n8cfg, validate=False)
        self._init_idx: dict = {}
        self._side_streams: dict = {}

    def _side_stream(self, device: torch.device) -> torch.cuda.Stream:
        s = self._side_streams.get(device)
        if s is None:
            s = torch.cuda.Stream(device=device)  # default priority
            self._side_streams[device] = s
        return s

    def _init_centroids(self, x: torch.Tensor, k: int, seed: int) -> torch.Tensor:
        bh, n, _ = x.shape
        key = (n, k, seed, x.device)
        idx = self._init_idx.get(key)
        if idx is None:
            idx = first_k_indices(n, k, seed).to(torch.int32).to(x.device)
            self._init_idx[key] = idx
        return gather_rows(x, idx.unsqueeze(0).expand(bh, -1))

    def route(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, timings: LayerTimings | None = None,
              *, materialize_kv: bool = True):
        """q, k, v [B, H, N, D] bf16 -> (N8V6Route, q sorted indices).

        With materialize_kv False the route carries no permuted K/V copies
        (k_permuted / v_permuted are None): forward() reads K and V through the
        key sort index instead."""
        route, q_idx, _ = self._route(q, k, v, timings, materialize_kv=materialize_kv, with_probes=False)
        return route, q_idx

    def _route(self, q, k, v, timings, *, materialize_kv: bool, with_probes: bool):
        """route() plus, with with_probes, the repair's base-independent part (probe rows
        and the dense attention of the probe queries), which needs only Q's clusters.

        With overlap_streams, Q's Lloyd loop and that probe part run on a side stream
        while K's Lloyd loop runs on the caller's stream; then the top-p map runs on the
        side stream beside the K/V permutation on the caller's, which waits for it before
        returning, so every later stage sees both."""
        cfg = self.config
        _lib.require_gpu(q, k, v, what="SparsePRAttention")
        B, H, N, D = q.shape
        bh = B * H
        qf = q.reshape(bh, N, D).contiguous()
        kf = k.reshape(bh, N, D).contiguous()
        route = N8V6Route(
            q_labels=None, k_labels=None, q_cluster_sizes=None, k_cluster_sizes=None, video_dynamic_map=None,
            q_role_features=qf, k_permuted=None, v_permuted=None, k_sorted_indices=None, base_video_density=None,
            q_kmeans_iters=0, k_kmeans_iters=0)

        def q_side():
            qres = lloyd(qf, cfg.num_q_centroids, cfg.kmeans_iters, 0.0,
                         self._init_centroids(qf, cfg.num_q_centroids, cfg.init_seed),
                         x_sq_mode=cfg.x_sq_mode, want_mean32=True)
            route.q_labels, route.q_cluster_sizes = qres.labels, qres.sizes
            route.q_role_centers, route.q_kmeans_iters = qres.mean32, qres.iters
            probes = self.n8.repair_probes(q, k, v, route) if with_probes else None
            return qres, probes

        main = torch.cuda.current_stream(q.device)
        overlap = cfg.overlap_streams if cfg.overlap_streams is not None else bh * N >= OVERLAP_MIN_TOKEN_HEADS
        side = self._side_stream(q.device) if overlap else None
        if side is not None:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                qres, probes = q_side()
        else:
            qres, probes = q_side()
        kres = lloyd(kf, cfg.num_k_centroids, cfg.kmeans_iters, 0.0,
                     self._init_centroids(kf, cfg.num_k_centroids, cfg.init_seed + 1), x_sq_mode=cfg.x_sq_mode)
        if side is not None:
            main.wait_stream(side)
            # made on the side stream, read on this one: keep the allocator from handing
            # their memory back to the side stream before this stream is done with them
            shared = [qres.labels, qres.centroids, qres.sizes, qres.sorted_idx, qres.offsets, qres.mean32]
            if probes is not None:
                shared += [probes[0], probes[1], probes[2]]
            for t in shared:
                if t is not None:
                    t.record_stream(main)
        if timings is not None:
            timings.mark("kmeans")
        self.last_centroids = (qres.centroids, kres.centroids)

        def select():
            dmap = topp_map(qres.centroids, kres.centroids, kres.sizes, cfg.top_p, cfg.min_kc_ratio)
            return dmap, density(dmap, qres.sizes, kres.sizes).mean()  # device scalar: no host sync

        if side is not None:
            # the map (latency-bound) on the side stream beside the K/V permutation (HBM-bound)
            side.wait_stream(main)
            for t in (kres.centroids, kres.sizes):
                t.record_stream(side)
            with torch.cuda.stream(side):
                dmap, dens = select()
        else:
            dmap, dens = select()
        if materialize_kv:
            from .kernels.permute import permute_tensor_by_labels_triton

            route.k_permuted, _ = permute_tensor_by_labels_triton(k, None, 2, sorted_indices=kres.sorted_idx)
            route.v_permuted, _ = permute_tensor_by_labels_triton(v, None, 2, sorted_indices=kres.sorted_idx)
        if side is not None:
            main.wait_stream(side)
            dmap.record_stream(main)
            dens.record_stream(main)
        if timings is not None:
            timings.mark("select")
        route.k_labels, route.k_cluster_sizes, route.k_sorted_indices = kres.labels, kres.sizes, kres.sorted_idx
        route.video_dynamic_map, route.k_kmeans_iters = dmap, kres.iters
        route.base_video_density = dens
        return route, qres.sorted_idx, probes

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, timings: LayerTimings | None = None):
        """Sparse attention output [B, H, N, D] bf16 (with repair unless disabled)."""
        cfg = self.config
        B, H, N, D = q.shape
        bh = B * H
        if timings is not None:
            timings.mark("start")
        route, q_idx, probes = self._route(q, k, v, timings, materialize_kv=True, with_probes=cfg.repair)
        plan = plan_block_sparse(route.video_dynamic_map, route.q_cluster_sizes, route.k_cluster_sizes, N)
        if timings is not None:
            timings.mark("plan")
        # The Q permutation and the output's inverse permutation (hunyuanvideo.py:189-231)
        # are fused into the attention through q_index: q and base stay in token order.
        # K and V are read from their cluster-sorted copies: contiguous key ranges
        # keep the key stream's cache locality (gathering them through
        # k_sorted_indices instead costs more attention time than the copies).
        base = block_sparse_attention(q.reshape(bh, N, D), route.k_permuted.reshape(bh, N, D),
                                      route.v_permuted.reshape(bh, N, D), route.video_dynamic_map,
                                      route.q_cluster_sizes, route.k_cluster_sizes, plan=plan,
                                      q_index=q_idx).view(B, H, N, D)
        if timings is not None:
            timings.mark("attention")
        self.last_route = route
        if not cfg.repair:
            return base
        out, info = self.n8.repair_finish(base, probes, route)
        self.last_repair_info = info
        if timings is not None:
            timings.mark("repair")
        return out

    __call__ = forward

    def graphed(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, warmup: int = 2) -> "LayerGraph":
        """This layer captured as a HIP graph for inputs of q's, k's and v's shapes."""
        return LayerGraph(self, q, k, v, warmup)


class LayerGraph:
    """One SparsePR layer call captured as a HIP graph over input buffers of its own.

    Every kernel of the layer (both streams' Lloyd loops, the map, the permutation, the
    plan, the attention and the repair) is recorded once; a call copies new Q, K, V into
    the captured buffers and replays the graph, so the host launches one graph instead of
    about a hundred kernels.  The result is the same bits as an eager call on the same
    inputs.  `out` is overwritten by the next replay: clone it to keep it.  Calls on one
    layer (graphed or eager) stay stream ordered; the repair's last finite state carries
    over between them as in eager calls."""

    def __init__(self, layer: "SparsePRAttention", q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 warmup: int = 2):
        _lib.require_gpu(q, k, v, what="LayerGraph")
        self.layer = layer
        self.q, self.k, self.v = q.clone(), k.clone(), v.clone()
        dev = q.device
        cur = torch.cuda.current_stream(dev)
        # warm-up calls make every lazily built buffer and cache before the capture
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                layer(self.q, self.k, self.v)
        cur.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = layer(self.q, self.k, self.v)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.out

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        if q.shape != self.q.shape or k.shape != self.k.shape or v.shape != self.v.shape:
            raise RuntimeError(f"LayerGraph was captured for Q/K/V {tuple(self.q.shape)}; got {tuple(q.shape)}, "
                               f"{tuple(k.shape)}, {tuple(v.shape)}")
        self.q.copy_(q)
        self.k.copy_(k)
        self.v.copy_(v)
        return self.replay()


def kept_pair_flops(route: N8V6Route, head_dim: int) -> torch.Tensor:
    """Executed attention flops: 4 * D * sum over kept (a, c) of |Q_a| |K_c| (device scalar)."""
    qs = route.q_cluster_sizes.to(torch.float64)
    ks = route.k_cluster_sizes.to(torch.float64)
    m = route.video_dynamic_map.to(torch.float64)
    pairs = torch.einsum("hq,hqk,hk->", qs, m, ks)
    return 4.0 * head_dim * pairs


def dense_flops(heads: int, tokens: int, head_dim: int) -> float:
    return 4.0 * heads * tokens * tokens * head_dim


__all__ = ["SparsePRAttention", "SparsePRConfig", "LayerTimings", "kept_pair_flops", "dense_flops"]
