#!/usr/bin/env python3
"""Benchmark: one SparsePR attention layer at the HunyuanVideo shape on one MI355X.

Workload: batch 1, 24 heads, 118,800 tokens (33 x 45 x 80),
head_dim 128, bf16; flash k-means with 128 Q-clusters and 512 K-clusters
(5 Lloyd iterations, seeded first-k init), top-p 0.9 cluster-pair selection,
block-sparse attention, N8 repair with 128 probes.  Synthetic frame-correlated
Gaussian-mixture Q/K/V (400 components), generated on the device before timing.

One step = one full layer call (route + attention + repair) on inputs resident
in HBM.  Prints ONE JSON line.  `roofline` describes the dominant kernel (the
block-sparse attention, MFMA-bound): algorithmic flops = 4 * D * sum of kept
|Q_a| * |K_c| pairs, divided by the kernel's average duration measured with HIP
events around its launch on the stream it runs on.  `cpu_baseline` times the
CPU oracle (numpy, the reference algorithm restated) on a bounded sample
(the first head of the same inputs), scaled to ms per layer.
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
    ap.add_argument("--top-p", type=float, default=0.9)
    ap.add_argument("--no-repair", action="store_true", help="route + attention only (sweep use)")
    ap.add_argument("--cpu-heads", type=int, default=1, help="heads in the CPU-oracle sample (0 = skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["attention", "copy", "svg_ear", "role_proj"], default=None,
                    help="profiling aids: 'attention' routes once, then times only the block-sparse attention "
                         "kernel for --steps launches; 'copy' runs --steps plain 512 MiB device copies (the "
                         "calibration kernel for the HBM traffic counters); 'svg_ear' routes once, then times "
                         "the N8 value-error routing scores (N8's default selector) on the routed clusters; "
                         "'role_proj' times N8's Q role projection (rank 64) over the C4 Q")
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


def cpu_baseline(q, k, v, cfg, heads: int):
    """Time the CPU oracle's layer on `heads` heads of the same inputs."""
    import numpy as np

    from oracle import sparsepr_oracle as orc

    try:
        from threadpoolctl import threadpool_info

        threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    qn = q[0, :heads].float().cpu().numpy()
    kn = k[0, :heads].float().cpu().numpy()
    vn = v[0, :heads].float().cpu().numpy()
    ocfg = orc.LayerConfig(q_clusters=cfg.num_q_centroids, k_clusters=cfg.num_k_centroids,
                           kmeans_iters=cfg.kmeans_iters, top_p=cfg.top_p, probes=cfg.probe_rows,
                           init_seed=cfg.init_seed)
    stages: dict = {}
    t0 = time.perf_counter()
    orc.sparsepr_layer(qn, kn, vn, ocfg, timings=stages)
    secs = time.perf_counter() - t0
    total_heads = q.shape[1]
    return {
        "value": round(secs * 1e3 * total_heads / heads, 1),
        "unit": "ms/layer",
        "cores": int(threads),
        "kind": "port",
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
    layer = SparsePRAttention(SparsePRConfig(top_p=args.top_p, repair=False))
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
    layer = SparsePRAttention(SparsePRConfig(top_p=args.top_p, repair=False))
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
    import torch

    from sparsepr_amd import synthetic
    from sparsepr_amd.layer import LayerTimings, SparsePRAttention, SparsePRConfig, dense_flops, kept_pair_flops

    torch.cuda.set_device(0)
    shape = synthetic.HUNYUAN
    q, k, v = synthetic.frame_gmm_qkv(shape, device="cuda", **GEN)
    cfg = SparsePRConfig(num_q_centroids=128, num_k_centroids=512, kmeans_iters=5, top_p=args.top_p,
                         probe_rows=128, repair=not args.no_repair)
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
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps

    names = list(marks[0].events)
    stage_ms = {b: round(sum(m.ms(a, b) for m in marks) / len(marks), 3) for a, b in zip(names[:-1], names[1:])}
    attn_ms = sum(m.ms("plan", "attention") for m in marks) / len(marks)
    route = layer.last_route
    kept = float(kept_pair_flops(route, shape.dim).item())
    dens = float(route.base_video_density.item())
    achieved = kept / (attn_ms * 1e-3) / 1e12
    traffic = traffic_from_profiles()

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
            "workload": "C4 HunyuanVideo-shaped SparsePR layer: 1x24x118800x128 bf16, Qc=128, Kc=512, "
                        f"5 Lloyd iters, top-p {args.top_p}, " + ("no repair" if args.no_repair else "128 probes"),
            "heads": shape.heads, "tokens": shape.tokens, "head_dim": shape.dim,
            "kept_pair_density": round(dens, 4),
            "kept_attention_tflop": round(kept / 1e12, 3),
            "dense_attention_tflop": round(dense_flops(shape.heads, shape.tokens, shape.dim) / 1e12, 1),
            "generator": GEN,
        },
        "stages_ms": stage_ms,
        "roofline": {
            "kernel": "attn_pipe_kernel (D=128 block-sparse attention)",
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "kernel_ms": round(attn_ms, 3),
        },
    }
    if not args.no_cpu_baseline and args.cpu_heads > 0:
        result["cpu_baseline"] = cpu_baseline(q, k, v, cfg, args.cpu_heads)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
