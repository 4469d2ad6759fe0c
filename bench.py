#!/usr/bin/env python3
"""Benchmark: one SparsePR attention layer at the BASELINE shapes on one MI355X.

Default workload (the headline): batch 1, 24 heads, 118,800 tokens
(33 x 45 x 80), head_dim 128, bf16; flash k-means with 128 Q-clusters and 512 K-clusters
(5 Lloyd iterations, seeded first-k init), top-p 0.9 cluster-pair selection, block-sparse
attention, N8 repair with 128 probes.  Synthetic frame-correlated Gaussian-mixture Q/K/V
(400 components), generated on the device before timing.

--config selects another BASELINE configuration:
  c1  the CPU-runnable case (2 x 4,096 x 64, Qc 32, Kc 64, 10 iterations, 64 probes);
  c2  standalone batched k-means (24 x 118,800 x 128, K 256, 5 iterations);
  c3  Wan2.2 (40 x 32,760 x 128, Qc 100, Kc 500, 128 probes);
  c4  HunyuanVideo (the default);
  c5  Cosmos2.5 (40 x 84,480 x 128, Qc 128, Kc 512): one line per top-p in
      {0.7, 0.8, 0.9, 0.95} x repair on/off (or the --top-p / --no-repair point).

One step = one full layer call (route + attention + repair) on inputs resident in HBM
(c2: one Lloyd loop).  Each line carries `roofline` for the dominant kernel, measured
with HIP events around its launches on the stream it runs on.  `cpu_baseline` is the
CPU oracle (numpy, the reference algorithm restated) at BASELINE config 1, median of 5
runs after 1 warm-up with the per-stage split, in the same process as the GPU run;
`cpu_baseline_same_workload` times one head of the measured workload itself.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "SparsePR attn ms/layer + % MFMA/HBM roofline at 118,800-token video shape"
MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0
GEN = dict(seed=0, amp=2.3, qk_corr=0.1, step_std=0.1, noise_std=0.3)


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", choices=["c1", "c2", "c3", "c4", "c5"], default="c4",
                    help="BASELINE configuration (c4, the HunyuanVideo layer, is the headline)")
    ap.add_argument("--amp", type=float, default=None,
                    help="component-mean amplitude of the generator (default 2.3; 1.0 is the literal "
                         "means ~N(0, 1) of the BASELINE description)")
    ap.add_argument("--top-p", type=float, default=None)
    ap.add_argument("--no-repair", action="store_true", help="route + attention only (sweep use)")
    ap.add_argument("--graph", action="store_true",
                    help="time the layer captured as a HIP graph (sparsepr_amd.layer.LayerGraph) over the same "
                         "inputs: `value` is the replay time; stages and roofline come from the eager calls")
    ap.add_argument("--one-stream", action="store_true",
                    help="run the whole layer on one stream (by default Q's k-means and the repair's probe "
                         "part run on a second stream beside K's k-means)")
    ap.add_argument("--cpu-heads", type=int, default=1, help="heads in the CPU-oracle sample (0 = skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["attention", "copy", "svg_ear", "role_proj", "n8_route", "qkv"], default=None,
                    help="profiling aids: 'attention' routes once, then times only the block-sparse attention "
                         "kernel for --steps launches; 'copy' runs --steps plain 512 MiB device copies (the "
                         "calibration kernel for the HBM traffic counters); 'svg_ear' routes once, then times "
                         "the N8 value-error routing scores (N8's default selector) on the routed clusters; "
                         "'role_proj' times N8's Q role projection (rank 64) over the C4 Q; 'n8_route' times the "
                         "HunyuanVideo adapter's N8 step (route, attention, repair) at the C4 shape; 'qkv' times "
                         "the Wan and Cosmos2.5 QKV norm + RoPE fusions at the C3 / C5 shapes")
    return ap.parse_args()


def traffic_from_profiles():
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary, if any."""
    f = ROOT / "profiles" / "attention_c4_hbm_traffic.json"
    if not f.exists():
        return None
    try:
        return float(json.loads(f.read_text())["bytes_per_launch"])
    except Exception:
        return None


def _cpu_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return int(max([p.get("num_threads", 1) for p in threadpool_info()] or [1]))
    except Exception:
        return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def _oracle_cfg(cfg):
    from oracle import sparsepr_oracle as orc

    return orc.LayerConfig(q_clusters=cfg.num_q_centroids, k_clusters=cfg.num_k_centroids,
                           kmeans_iters=cfg.kmeans_iters, top_p=cfg.top_p, probes=cfg.probe_rows,
                           init_seed=cfg.init_seed)


def cpu_baseline_c1(runs: int = 5):
    """BASELINE config 1 on the CPU oracle, as the CPU baseline plan specifies: fp32, median of
    `runs` runs after one warm-up, per-stage split; the block-sparse attention both as the
    loop-faithful restatement of dynamic_block_sparse_fwd_torch and as the vectorized
    masked-dense variant.  Also times the GPU layer on the same inputs (bf16) in this process."""
    import numpy as np
    import torch

    from oracle import sparsepr_oracle as orc
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRAttention

    c1 = _layer_configs()["c1"]
    shape, gen, cfg = c1["shape"], c1["gen"], c1["cfg"]
    q, k, v = synthetic.frame_gmm_qkv(shape, device="cpu", dtype=torch.float32, **gen)
    qn, kn, vn = (t[0].numpy() for t in (q, k, v))
    ocfg = _oracle_cfg(cfg)
    torch.set_num_threads(os.cpu_count() or 1)
    res = {}
    for attention in ("loop", "dense"):
        totals, stages = [], []
        for i in range(runs + 1):
            st: dict = {}
            t0 = time.perf_counter()
            orc.sparsepr_layer(qn, kn, vn, ocfg, timings=st, bf16=False, attention=attention)
            if i > 0:  # the first run is the warm-up
                totals.append((time.perf_counter() - t0) * 1e3)
                stages.append(st)
        med = int(np.argsort(totals)[len(totals) // 2])
        res[attention] = (float(np.median(totals)), {k: round(v, 2) for k, v in stages[med].items()})
    # the GPU layer on the same inputs (bf16: the kernels' input type)
    qg, kg, vg = (t.to("cuda", torch.bfloat16) for t in (q, k, v))
    layer = SparsePRAttention(cfg)
    for _ in range(3):
        layer(qg, kg, vg)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        layer(qg, kg, vg)
    torch.cuda.synchronize()
    gpu_ms = (time.perf_counter() - t0) * 1e3 / 20
    loop_ms, loop_st = res["loop"]
    dense_ms, dense_st = res["dense"]
    return {
        "value": round(loop_ms, 2),
        "unit": "ms/layer at BASELINE config 1",
        "cores": _cpu_threads(),
        "kind": "port",
        "sample": ("BASELINE config 1 (1 x 2 x 4,096 x 64 fp32, Qc 32, Kc 64, 10 Lloyd iterations, top-p 0.9, "
                   f"64 probes) on the CPU oracle, median of {runs} runs after 1 warm-up, loop-faithful "
                   "block-sparse attention"),
        "stages_ms": loop_st,
        "vectorized_attention_variant": {"value": round(dense_ms, 2), "stages_ms": dense_st},
        "gpu_ms_same_inputs_bf16": round(gpu_ms, 3),
    }


def cpu_baseline_slice(q, k, v, cfg, heads: int):
    """The CPU oracle's layer on `heads` heads of the measured inputs (the heads are
    independent, so the layer's CPU time is this slice's times H / heads, reported as such)."""
    from oracle import sparsepr_oracle as orc

    qn = q[0, :heads].float().cpu().numpy()
    kn = k[0, :heads].float().cpu().numpy()
    vn = v[0, :heads].float().cpu().numpy()
    stages: dict = {}
    t0 = time.perf_counter()
    orc.sparsepr_layer(qn, kn, vn, _oracle_cfg(cfg), timings=stages)
    secs = time.perf_counter() - t0
    total_heads = q.shape[1]
    return {
        "value": round(secs * 1e3 * total_heads / heads, 1),
        "unit": "ms/layer",
        "cores": _cpu_threads(),
        "kind": "port",
        "slice_ms": round(secs * 1e3, 1),
        "sample": (f"CPU oracle (numpy restatement: k-means, top-p map, loop-faithful block-sparse attention, "
                   f"N8 repair) on {heads} of {total_heads} heads of the same inputs, {secs:.1f} s, scaled x"
                   f"{total_heads / heads:g}; stage ms: " + ", ".join(f"{k}={v:.0f}" for k, v in stages.items())),
    }


def only_copy(args):
    """--steps device copies of 512 MiB (read 512 MiB + write 512 MiB per launch)."""
    import torch

    n = 256 * 1024 * 1024
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    print(json.dumps({"copy_bytes_per_launch": n * 2, "ms_per_copy": round(ms, 4),
                      "gbs_read_plus_write": round(2 * n * 2 / ms / 1e6, 1)}), flush=True)


def only_attention(args):
    """Route the C4 inputs once, then time --steps launches of the block-sparse attention alone."""
    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.kernels.attention import block_sparse_attention, plan_block_sparse
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig, kept_pair_flops

    shape = synthetic.HUNYUAN
    q, k, v = synthetic.frame_gmm_qkv(shape, device="cuda", **GEN)
    layer = SparsePRAttention(SparsePRConfig(top_p=args.top_p or 0.9, repair=False))
    route, q_idx = layer.route(q, k, v)
    B, H, N, D = q.shape
    plan = plan_block_sparse(route.video_dynamic_map, route.q_cluster_sizes, route.k_cluster_sizes, N)

    def run():  # the layer's call: token-order q read through its sort index, cluster-sorted K/V
        return block_sparse_attention(q.reshape(B * H, N, D), route.k_permuted.reshape(B * H, N, D),
                                      route.v_permuted.reshape(B * H, N, D), route.video_dynamic_map,
                                      route.q_cluster_sizes, route.k_cluster_sizes, plan=plan, q_index=q_idx)

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    flops = float(kept_pair_flops(route, D).item())
    print(json.dumps({"kernel": "attn_pipe_kernel", "ms_per_launch": round(ms, 3),
                      "tflops": round(flops / ms / 1e9, 1), "frac": round(flops / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
                      "density": round(float(route.base_video_density.item()), 4)}), flush=True)


def only_svg_ear(args):
    """Route the C4 inputs once, then time --steps launches of the SVG-EAR value-error routing
    scores (all 24 heads x 128 query centroids x 512 key clusters over the cluster-sorted K/V).
    Algorithmic HBM bytes per launch: K and V read once (2 * BH * N * D * 2) plus the
    centroids and the score matrix; algorithmic flops: 2 * BH * Qc * N * D (token logits)."""
    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.kernels.svg_ear import svg_ear_value_error_scores_triton
    from sparsepr_amd.layer import SparsePRAttention, SparsePRConfig

    shape = synthetic.HUNYUAN
    q, k, v = synthetic.frame_gmm_qkv(shape, device="cuda", **GEN)
    layer = SparsePRAttention(SparsePRConfig(top_p=args.top_p or 0.9, repair=False))
    route, _ = layer.route(q, k, v)
    B, H, N, D = q.shape
    bh = B * H
    qc = layer.last_centroids[0].float().reshape(bh, -1, D).contiguous()
    kc = layer.last_centroids[1].float().reshape(bh, -1, D).contiguous()
    sizes = route.k_cluster_sizes.reshape(bh, -1).to(torch.int32).contiguous()
    ks, vs = route.k_permuted.reshape(bh, N, D), route.v_permuted.reshape(bh, N, D)
    # value centroids: per-cluster means of the sorted V (prefix sums over the runs)
    ends = sizes.long().cumsum(1)
    csum = torch.nn.functional.pad(vs.float().cumsum(1), (0, 0, 1, 0))
    vc = ((csum.gather(1, ends[..., None].expand(-1, -1, D))
           - csum.gather(1, (ends - sizes.long())[..., None].expand(-1, -1, D)))
          / sizes.clamp_min(1)[..., None].float()).contiguous()
    del csum

    def run():
        return svg_ear_value_error_scores_triton(qcentroids=qc, k_sorted=ks, v_sorted=vs, kcentroids=kc,
                                                 vcentroids=vc, kcluster_sizes=sizes, gqa_group=1)

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        scores = run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    qn, kn = qc.shape[1], kc.shape[1]
    nbytes = 2 * bh * N * D * 2 + (qc.numel() + kc.numel() + vc.numel() + scores.numel()) * 4
    flops = 2.0 * bh * qn * N * D
    gbs = nbytes / ms / 1e6
    print(json.dumps({"kernel": "svg_ear_score_kernel<value>", "ms_per_launch": round(ms, 4),
                      "config": {"bh": bh, "tokens": N, "q_clusters": qn, "k_clusters": kn},
                      "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes},
                      "tflops": round(flops / ms / 1e9, 1),
                      "finite_scores": round(float(torch.isfinite(scores).float().mean().item()), 4)}), flush=True)


def only_role_proj(args):
    """--steps launches of the Q role projection + row RMS normalisation at the C4 shape
    (24 heads x 118,800 tokens, D = 128, rank 64).  Algorithmic HBM bytes per launch: Q read
    once (bf16) + the fp32 features written once (+ the factors)."""
    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.kernels.role_projection import role_projection_rms_triton

    shape = synthetic.HUNYUAN
    q, _, _ = synthetic.frame_gmm_qkv(shape, device="cuda", **GEN)
    B, H, N, D = q.shape
    x = q.reshape(B * H, N, D)
    g = torch.Generator(device="cuda").manual_seed(1)
    factor = torch.randn((B * H, D, 64), device="cuda", generator=g) / D ** 0.5
    out = torch.empty((B * H, N, 64), device="cuda")
    for _ in range(args.warmup):
        role_projection_rms_triton(x, factor, out=out)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        role_projection_rms_triton(x, factor, out=out)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    nbytes = x.numel() * 2 + out.numel() * 4 + factor.numel() * 4
    gbs = nbytes / ms / 1e6
    print(json.dumps({"kernel": "role_projection_kernel<128, 2>", "ms_per_launch": round(ms, 4),
                      "config": {"bh": B * H, "tokens": N, "head_dim": D, "rank": 64},
                      "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes}}), flush=True)


def only_n8_route(args):
    """The HunyuanVideo adapter's N8 step at the C4 shape (hunyuanvideo.py:160-239) with the
    default N8V6Config (300 Q / 1000 K clusters, ranks 64 / 48, fixed density 0.22, 64 probes):
    route (role metrics, warm factors, role-space k-means, centroids, K/V permute, SVG-EAR
    scores, exact budget selector), query permute, padded block-sparse attention over the
    118,800 video + 256 text tokens (77 prompt), inverse permute, repair.  Warm-up includes the
    cold call (25 Lloyd iterations); the timed steps are the warm calls of a denoising loop
    (2 iterations from the previous centroids).  Stage times come from one extra call with
    the route's synchronising profile marks; the attention is timed with HIP events on the
    stream it is launched on, inside the timed steps."""
    import torch
    import torch.nn.functional as F

    from sparsepr_amd import synthetic
    from sparsepr_amd.kernels.permute import apply_inverse_permutation_triton, permute_tensor_by_labels_triton
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    shape = synthetic.HUNYUAN
    text, prompt = 256, 77
    qv, kv, vv = synthetic.frame_gmm_qkv(shape, device=dev, **GEN)
    B, H, Nv, D = qv.shape
    g = torch.Generator(device=dev).manual_seed(5)
    query, key, value = (torch.cat((a, (0.8 * torch.randn((B, H, text, D), device=dev, generator=g)).to(a.dtype)), 2)
                         for a in (qv, kv, vv))
    cfg = N8V6Config()
    core = N8V6Core(cfg)
    text_idx = torch.arange(Nv, Nv + text, device=dev, dtype=torch.int32).expand(B * H, -1)
    sizes_tail = torch.tensor([prompt, text - prompt], device=dev, dtype=torch.long)
    attn_events = []

    def step(ev=None):
        route = core.route(qv, kv, vv, always_attended_keys=prompt, total_key_tokens=Nv + prompt,
                           k_full_source=key, v_full_source=value)
        q_order = torch.argsort(route.q_labels, dim=-1, stable=True).to(torch.int32)
        q_perm, _ = permute_tensor_by_labels_triton(query, None, dim=2,
                                                    sorted_indices=torch.cat((q_order, text_idx), 1).contiguous())
        qc, kc = route.video_dynamic_map.shape[-2:]
        block_map = F.pad(route.video_dynamic_map.view(B, H, qc, kc), (0, 2, 0, 2), value=False)
        block_map[:, :, :-1, -2] = True
        block_map[:, :, -2, :-1] = True
        block_map[:, :, -1, -1] = True
        qs = torch.cat((route.q_cluster_sizes.view(B, H, qc), sizes_tail.expand(B, H, 2)), 2)
        ks = torch.cat((route.k_cluster_sizes.view(B, H, kc), sizes_tail.expand(B, H, 2)), 2)
        if ev is not None:
            ev[0].record()
        out_perm = dynamic_block_sparse_fwd_flashinfer(q_perm, route.k_permuted, route.v_permuted, block_map, qs, ks,
                                                       is_cpu=False)
        if ev is not None:
            ev[1].record()
        base_video = apply_inverse_permutation_triton(out_perm[:, :, :Nv], q_order, dim=2)
        repaired, info = core.repair(base_video, qv, key[:, :, :Nv + prompt], value[:, :, :Nv + prompt], route)
        return route, block_map, qs, ks, info

    for _ in range(max(args.warmup, 1)):  # the first call is the cold one
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        attn_events.append(ev)
        route, block_map, qs, ks, info = step(ev)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    attn_ms = sum(a.elapsed_time(b) for a, b in attn_events) / len(attn_events)
    kept = float((block_map.float() * qs[..., :, None].float() * ks[..., None, :].float()).sum().item()) * 4 * D
    # one extra call with the route's stage marks (synchronising, so not in the timed steps)
    core.profile_breakdown_active = True
    t1 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    profiled_ms = (time.perf_counter() - t1) * 1e3
    core.profile_breakdown_active = False
    stages = {k[len("n8_route_"):-3]: round(v, 3) for k, v in core.last_route_profile.items()
              if k.startswith("n8_route_") and k.endswith("_ms")}
    bh, tot = B * H, Nv + text
    # algorithmic HBM bytes of the streaming stages (bf16 Q/K/V rows, fp32 role features)
    stage_bytes = {
        "kv_projection_init": bh * Nv * (D * 2 + cfg.role_k_rank * 4),
        "kv_centroids": bh * Nv * (2 * D * 2 + 4),
        "q_projection_init": bh * Nv * (D * 2 + cfg.role_q_rank * 4),
        "q_centroids": bh * Nv * (D * 2 + 4),
        "kv_permute": bh * tot * (4 * D * 2 + 4),
        "selector_scores": bh * tot * 2 * D * 2,
    }
    stage_roofline = {name: {"ms": stages[name], "gbs": round(b / stages[name] / 1e6, 1),
                             "hbm_frac": round(b / stages[name] / 1e6 / HBM_PEAK_GBS, 4)}
                      for name, b in stage_bytes.items() if stages.get(name)}
    achieved = kept / (attn_ms * 1e-3) / 1e12
    print(json.dumps({
        "metric": "N8 (HunyuanVideo adapter) layer ms: route + padded block-sparse attention + repair",
        "value": round(ms, 3), "unit": "ms/layer", "n_gpus": 1, "steps": args.steps, "warmup": max(args.warmup, 1),
        "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (frame-correlated Gaussian mixture video + Gaussian text, seeded, on device)",
        "config": {"workload": "C4-shaped HunyuanVideo N8 step: 1x24x(118800 video + 256 text, 77 prompt)x128 bf16, "
                               "default N8V6Config (Qc 300, Kc 1000, ranks 64/48, density 0.22, 64 probes), warm calls",
                   "q_kmeans_iters": int(route.q_kmeans_iters), "k_kmeans_iters": int(route.k_kmeans_iters),
                   "base_video_density": round(float(route.base_video_density), 4),
                   "effective_video_density": round(float(info["effective_video_density"]), 4),
                   "kept_attention_tflop": round(kept / 1e12, 3), "generator": GEN},
        "stages_ms": {"route_profiled_call_ms": round(profiled_ms, 3), **stages},
        "stage_roofline": stage_roofline,
        "roofline": {"kernel": "attn_pipe_kernel (padded N8 map)", "bound": "mfma", "achieved": round(achieved, 1),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel_ms": round(attn_ms, 3)},
    }), flush=True)


def only_qkv(args):
    """The model-edge fusions at their models' shapes: Wan's Q/K RMSNorm + complex RoPE + BHLD
    layout at the C3 shape (1 x 32,760 x 40 heads x 128) and Cosmos2.5's per-head RMSNorm +
    rotate-half RoPE at the C5 shape (1 x 84,480 x 40 x 128), bf16.  One line per fusion,
    HBM roofline over the algorithmic bytes (Q, K, V read and written once, plus the RoPE
    table), timed with HIP events on the stream the kernel runs on."""
    import torch

    from sparsepr_amd.kernels.n8_extension import cosmos25_qkv_norm_rope_bshd, wan_qkv_norm_rope_layout

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    heads, d = 40, 128
    c = heads * d
    bf = torch.bfloat16
    cases = []
    tok = 32760
    qkv = [torch.randn((1, tok, c), device=dev, generator=g).to(bf) for _ in range(3)]
    w = [(1 + 0.1 * torch.randn(c, device=dev, generator=g)).to(bf) for _ in range(2)]
    ang = torch.rand((tok, d // 2), device=dev, generator=g) * 6.0
    fr, fi = torch.cos(ang).contiguous(), torch.sin(ang).contiguous()
    cases.append(("wan_qkv_kernel (Wan QKV RMSNorm + RoPE + BHLD layout)",
                  "C3 Wan2.2 shape: 1 x 32760 tokens x 40 heads x 128 bf16",
                  lambda: wan_qkv_norm_rope_layout(*qkv, *w, fr, fi, heads=heads, epsilon=1e-6),
                  6 * tok * c * 2 + tok * d * 4 + 2 * c * 2))
    tok2 = 84480
    qkv2 = [torch.randn((1, tok2, c), device=dev, generator=g).to(bf) for _ in range(3)]
    w2 = [1 + 0.1 * torch.randn(d, device=dev, generator=g) for _ in range(2)]
    ang2 = (torch.rand((tok2, 1, 1, d), device=dev, generator=g) * 40.0).contiguous()
    cases.append(("cosmos_qkv_kernel<bf16, 128> (Cosmos2.5 QKV RMSNorm + rotate-half RoPE)",
                  "C5 Cosmos-Predict2.5 shape: 1 x 84480 tokens x 40 heads x 128 bf16",
                  lambda: cosmos25_qkv_norm_rope_bshd(*qkv2, *w2, ang2, heads=heads, epsilon=1e-6),
                  6 * tok2 * c * 2 + tok2 * d * 4 + 2 * d * 4))
    for kernel, workload, run, nbytes in cases:
        for _ in range(max(args.warmup, 1)):
            run()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            run()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        gbs = nbytes / ms / 1e6
        print(json.dumps({
            "metric": "QKV norm + RoPE fusion ms per call + % HBM roofline", "value": round(ms, 4), "unit": "ms/call",
            "n_gpus": 1, "steps": args.steps, "warmup": max(args.warmup, 1), "ms_per_step": round(ms, 4),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (Gaussian Q/K/V, seeded, on device)", "config": {"workload": workload},
            "roofline": {"kernel": kernel, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": nbytes, "kernel_ms": round(ms, 4)},
        }), flush=True)


def _layer_configs():
    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import SparsePRConfig

    c1_gen = dict(seed=0, amp=1.0, step_std=0.0, noise_std=0.3, qk_corr=1.0)
    return {
        "c1": dict(shape=synthetic.CPU_SMALL, gen=c1_gen,
                   cfg=SparsePRConfig(num_q_centroids=32, num_k_centroids=64, kmeans_iters=10, top_p=0.9,
                                      probe_rows=64),
                   workload="C1 CPU-runnable SparsePR layer: 1x2x4096x64 (4 x 32 x 32), Qc=32, Kc=64, "
                            "10 Lloyd iters, top-p 0.9, 64 probes"),
        "c3": dict(shape=synthetic.WAN, gen=GEN,
                   cfg=SparsePRConfig(num_q_centroids=100, num_k_centroids=500, kmeans_iters=5, top_p=0.9,
                                      probe_rows=128),
                   workload="C3 Wan2.2-shaped SparsePR layer: 1x40x32760x128 bf16, Qc=100, Kc=500, "
                            "5 Lloyd iters, top-p 0.9, 128 probes"),
        "c4": dict(shape=synthetic.HUNYUAN, gen=GEN,
                   cfg=SparsePRConfig(num_q_centroids=128, num_k_centroids=512, kmeans_iters=5, top_p=0.9,
                                      probe_rows=128),
                   workload="C4 HunyuanVideo-shaped SparsePR layer: 1x24x118800x128 bf16, Qc=128, Kc=512, "
                            "5 Lloyd iters, top-p 0.9, 128 probes"),
        "c5": dict(shape=synthetic.COSMOS, gen=GEN,
                   cfg=SparsePRConfig(num_q_centroids=128, num_k_centroids=512, kmeans_iters=5, top_p=0.9,
                                      probe_rows=128),
                   workload="C5 Cosmos-Predict2.5-shaped SparsePR layer: 1x40x84480x128 bf16, Qc=128, Kc=512, "
                            "5 Lloyd iters"),
    }


def bench_layer(args, name, top_p=None, repair=True, amp=None, with_cpu=False):
    """Time `args.steps` layer calls after `args.warmup`; returns the JSON result dict."""
    import dataclasses

    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import LayerTimings, SparsePRAttention, dense_flops, kept_pair_flops

    spec = _layer_configs()[name]
    shape = spec["shape"]
    gen = dict(spec["gen"])
    if amp is not None:
        gen["amp"] = amp
    cfg = spec["cfg"]
    if top_p is not None:
        cfg = dataclasses.replace(cfg, top_p=top_p)
    cfg = dataclasses.replace(cfg, repair=repair, overlap_streams=False if args.one_stream else None)
    q, k, v = synthetic.frame_gmm_qkv(shape, device="cuda", **gen)
    layer = SparsePRAttention(cfg)
    for _ in range(args.warmup):
        layer(q, k, v)
    torch.cuda.synchronize()
    marks = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tm = LayerTimings()
        layer(q, k, v, timings=tm)
        marks.append(tm)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    eager_ms = ms_per_step
    if args.graph:
        g = layer.graphed(q, k, v)
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.replay()
        torch.cuda.synchronize()
        ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    names = list(marks[0].events)
    stage_ms = {b: round(sum(m.ms(a, b) for m in marks) / len(marks), 3) for a, b in zip(names[:-1], names[1:])}
    attn_ms = sum(m.ms("plan", "attention") for m in marks) / len(marks)
    route = layer.last_route
    kept = float(kept_pair_flops(route, shape.dim).item())
    dens = float(route.base_video_density.item())
    achieved = kept / (attn_ms * 1e-3) / 1e12
    heads, tokens, d = shape.heads, shape.tokens, shape.dim
    # algorithmic bytes of the attention: Q, K, V read once and O written once (bf16)
    attn_bytes = 4 * heads * tokens * d * 2
    workload = spec["workload"]
    if name == "c5":
        workload += f", top-p {cfg.top_p}, " + ("128 probes" if repair else "no repair")
    result = {
        "metric": METRIC,
        "value": round(ms_per_step, 3),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (frame-correlated Gaussian mixture, seeded, generated on device)",
        "config": {
            "workload": workload, "heads": heads, "tokens": tokens, "head_dim": d, "top_p": cfg.top_p,
            "repair": repair, "kept_pair_density": round(dens, 4),
            "kept_attention_tflop": round(kept / 1e12, 3),
            "dense_attention_tflop": round(dense_flops(heads, tokens, d) / 1e12, 2),
            "generator": gen,
        },
        "launch": "hip_graph_replay" if args.graph else "eager",
        "eager_ms_per_step": round(eager_ms, 3),
        "stages_ms": stage_ms,
        "roofline": {
            "kernel": "attn_pipe_kernel (D=128 block-sparse attention)" if d == 128
            else "attn_fwd_kernel<64> (D=64 block-sparse attention)",
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic_from_profiles() if name == "c4" and amp is None and cfg.top_p == 0.9 else None,
            "kernel_ms": round(attn_ms, 3),
            # the same launch against the HBM roof: its floor is the larger of the two times
            "hbm_floor_ms": round(attn_bytes / HBM_PEAK_GBS / 1e6, 3),
            "mfma_floor_ms": round(kept / MFMA_BF16_PEAK_TFLOPS / 1e9, 3),
        },
    }
    if with_cpu and not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_c1()
        if args.cpu_heads > 0 and name != "c1":
            result["cpu_baseline_same_workload"] = cpu_baseline_slice(q, k, v, cfg, args.cpu_heads)
    return result


def bench_kmeans_c2(args):
    """batched flash k-means, 24 x 118,800 x 128 bf16, K = 256, 5 Lloyd
    iterations from a seeded first-k init.  value = ms per Lloyd loop.  The rooflines time the
    assign (MFMA / HBM) and the centroid update (sort + mean, HBM) separately with HIP events."""
    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.flash_kmeans.kmeans_impl import X_SQ_BF16, centroid_update_sorted, euclid_assign, lloyd
    from sparsepr_amd.kernels.permute import argsort_labels

    B, N, D, K, iters = 24, 118800, 128, 256, 5
    x = synthetic.gmm_points(B, N, D, 256, seed=0, std=0.25, device="cuda")
    idx = synthetic.first_k_indices(N, K, 0).to("cuda")
    init = x[:, idx].contiguous()

    def run():
        return lloyd(x, K, iters, 0.0, init, x_sq_mode=X_SQ_BF16)

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # the assign alone (later iterations: cached squared norms) and the update alone
    x_sq = torch.empty((B, N), device="cuda")
    labels = euclid_assign(x, res.centroids, None, x_sq_mode=X_SQ_BF16, x_sq_out=x_sq)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    for _ in range(args.steps):
        euclid_assign(x, res.centroids, x_sq, x_sq_mode=X_SQ_BF16, out=labels)
    ev[1].record()
    ev[2].record()
    for _ in range(args.steps):
        si, sz, off = argsort_labels(labels, K)
        centroid_update_sorted(x, labels, res.centroids, sorted_idx=si, sizes=sz, offsets=off)
    ev[3].record()
    torch.cuda.synchronize()
    assign_ms = ev[0].elapsed_time(ev[1]) / args.steps
    update_ms = ev[2].elapsed_time(ev[3]) / args.steps
    a_flops = 2.0 * B * N * K * D
    a_bytes = B * N * D * 2 + B * N * 4 + B * K * D * 2
    u_bytes = B * N * D * 2 + B * N * 4 + B * K * D * 4
    return {
        "metric": "flash_kmeans batched Lloyd ms (5 iterations) + % MFMA/HBM roofline",
        "value": round(ms, 3),
        "unit": "ms/loop",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (256-component Gaussian mixture, std 0.25, Dirichlet(1) weights, seeded, on device)",
        "config": {"workload": "C2 standalone batched k-means: 24 x 118800 x 128 bf16, K=256, 5 Lloyd iters, "
                               "first-k init", "batch": B, "points": N, "dim": D, "clusters": K,
                   "iters": int(res.iters)},
        # K = 256: 256 flop per byte, below the ~312 flop/B ridge, so the HBM floor is the higher one
        "roofline": {"kernel": "kmeans_assign_resident_kernel<128> (K=256)", "bound": "hbm",
                     "achieved": round(a_bytes / assign_ms / 1e6, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(a_bytes / assign_ms / 1e6 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel_ms": round(assign_ms, 4),
                     "mfma_tflops": round(a_flops / assign_ms / 1e9, 1),
                     "mfma_frac": round(a_flops / assign_ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "roofline_update": {"kernel": "label sort + centroid_mean_kernel (K=256)", "bound": "hbm",
                            "achieved": round(u_bytes / update_ms / 1e6, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(u_bytes / update_ms / 1e6 / HBM_PEAK_GBS, 4),
                            "kernel_ms": round(update_ms, 4)},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards by head with no "
              "communication, see the design notes.", file=sys.stderr)
        sys.exit(2)
    if args.only == "copy":
        return only_copy(args)
    if args.only == "attention":
        return only_attention(args)
    if args.only == "svg_ear":
        return only_svg_ear(args)
    if args.only == "role_proj":
        return only_role_proj(args)
    if args.only == "n8_route":
        return only_n8_route(args)
    if args.only == "qkv":
        return only_qkv(args)
    import torch

    torch.cuda.set_device(0)
    if args.config == "c2":
        print(json.dumps(bench_kmeans_c2(args)), flush=True)
        return
    if args.config == "c5" and args.top_p is None and not args.no_repair:
        for repair in (True, False):
            for top_p in (0.7, 0.8, 0.9, 0.95):
                print(json.dumps(bench_layer(args, "c5", top_p=top_p, repair=repair, amp=args.amp)), flush=True)
        return
    res = bench_layer(args, args.config, top_p=args.top_p, repair=not args.no_repair, amp=args.amp,
                      with_cpu=args.config in ("c1", "c4"))
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
