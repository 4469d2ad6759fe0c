"""SVG-EAR routing scores on the HIP kernel of csrc/spr_svg_ear.hip.

Same names, keyword signatures, validation and error texts as the reference's
src/sparsepr/kernels/triton/svg_ear.py (attention_mass_scores_triton :372-450,
svg_ear_value_error_scores_triton :453-531,
svg_ear_grouped_value_error_scores_triton :534-600, svg_ear_compensation_triton
:603-678).  The Triton tiling
parameters (block_q, block_n, num_warps, num_stages) are validated as the
reference validates them and otherwise ignored: the HIP kernel has one tiling
(four waves per (query head, key cluster), 32-token chunks).  K and V must be
bf16 (the reference's callers pass the permuted bf16 activations); the query
centroids, K/V centroids and variances are read as fp32.  There is no CPU path.
"""

from __future__ import annotations

import torch

from .. import _lib

MODE_VALUE_ERROR = 0
MODE_ATTENTION_MASS = 1


def _check_tiling(block_q: int, block_n: int, num_warps: int, num_stages: int, what: str) -> None:
    if block_q not in {8, 16, 32} or block_n not in {16, 32, 64}:
        raise RuntimeError(f"{what} supports BQ={{8,16,32}}, BN={{16,32,64}}.")
    if num_warps not in {2, 4, 8} or num_stages not in {1, 2, 3}:
        raise RuntimeError(f"{what} supports warps={{2,4,8}}, stages={{1,2,3}}.")


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise RuntimeError(f"{name} must be bfloat16 for the HIP routing scores (got {t.dtype}).")
    return t.contiguous()


def _launch(mode: int, qcentroids, k_sorted, v_sorted, kcentroids, vcentroids, var_k_diag, jensen_var_cap,
            kcluster_sizes, gqa_group: int) -> torch.Tensor:
    dev = _lib.require_gpu(qcentroids, k_sorted, v_sorted, kcentroids, vcentroids, var_k_diag, kcluster_sizes,
                           what="SVG-EAR routing scores")
    q_heads, q_clusters, dim = qcentroids.shape
    kv_heads, stored_tokens, _ = k_sorted.shape
    k_clusters = int(kcluster_sizes.shape[1]) if mode == MODE_ATTENTION_MASS else int(kcentroids.shape[1])
    sizes = kcluster_sizes.to(device=dev, dtype=torch.int32)
    if sizes.ndim != 2 or sizes.shape[1] != k_clusters:
        raise RuntimeError(f"SVG-EAR cluster-size shape {tuple(sizes.shape)} does not match {k_clusters} clusters.")
    # the reference reads the offsets row of kv head qh // gqa_group (svg_ear.py:149-150), so
    # rows past kv_heads are never used
    if sizes.shape[0] < kv_heads:
        raise RuntimeError(f"SVG-EAR cluster sizes need {kv_heads} rows, got {tuple(sizes.shape)}.")
    # no host-side check of the values (it would synchronise): the kernel counts a negative
    # size as 0 and clamps every cluster's token range to the stored tokens
    sizes = sizes[:kv_heads].contiguous()
    q32 = qcentroids.float().contiguous()
    k16 = _bf16(k_sorted, "k_sorted")
    v16 = kc32 = vc32 = var32 = None
    if mode == MODE_VALUE_ERROR:
        v16 = _bf16(v_sorted, "v_sorted")
        if v16.shape != k16.shape:
            raise RuntimeError(f"SVG-EAR K/V shape mismatch: {tuple(k16.shape)} vs {tuple(v16.shape)}.")
        kc32 = kcentroids.float().contiguous()
        vc32 = vcentroids.float().contiguous()
        expected = (kv_heads, k_clusters, dim)
        if tuple(kc32.shape) != expected or tuple(vc32.shape) != expected:
            raise RuntimeError(f"SVG-EAR centroid shape mismatch: K={tuple(kc32.shape)}, V={tuple(vc32.shape)}, "
                               f"expected={expected}.")
        if var_k_diag is not None and jensen_var_cap > 0.0:
            var32 = var_k_diag.float().contiguous()
    scores = torch.empty((q_heads, q_clusters, k_clusters), device=dev, dtype=torch.float32)
    _lib.call("spr_svg_ear_scores", _lib.ptr(q32), _lib.ptr(k16), _lib.ptr(v16), _lib.ptr(kc32), _lib.ptr(vc32),
              _lib.ptr(var32), float(jensen_var_cap), _lib.ptr(sizes), q_heads, q_clusters, k_clusters, kv_heads,
              stored_tokens, dim, int(gqa_group), mode, _lib.ptr(scores), _lib.stream(dev))
    return scores


def attention_mass_scores_triton(
    *,
    qcentroids: torch.Tensor,
    k_sorted: torch.Tensor,
    kcluster_sizes: torch.Tensor,
    gqa_group: int,
    block_q: int = 16,
    block_n: int = 32,
    num_warps: int = 4,
    num_stages: int = 1,
    logical_tokens: int | None = None,
) -> torch.Tensor:
    """Exact token-key cluster mass scores, up to a rowwise constant (svg_ear.py:372-450)."""
    if not qcentroids.is_cuda:
        raise RuntimeError("attention_mass_scores_triton requires CUDA tensors.")
    q_heads, q_clusters, dim = qcentroids.shape
    kv_heads, stored_tokens, k_dim = k_sorted.shape
    tokens = stored_tokens if logical_tokens is None else int(logical_tokens)
    if kcluster_sizes.ndim != 2 or kcluster_sizes.shape[0] != kv_heads:
        raise RuntimeError(
            "Attention-mass cluster sizes must be [KVH,Ck], got "
            f"{tuple(kcluster_sizes.shape)}."
        )
    if dim != 128 or k_dim != dim:
        raise RuntimeError(f"Attention-mass routing requires DIM=128, got q={dim}, k={k_dim}.")
    if q_heads != kv_heads * gqa_group:
        raise RuntimeError(
            "Attention-mass routing GQA mismatch: "
            f"q_heads={q_heads}, kv_heads={kv_heads}, group={gqa_group}."
        )
    if tokens <= 0 or tokens > stored_tokens:
        raise RuntimeError(f"Attention-mass logical tokens {tokens} must be in [1,{stored_tokens}].")
    _check_tiling(block_q, block_n, num_warps, num_stages, "Attention-mass routing")
    return _launch(MODE_ATTENTION_MASS, qcentroids, k_sorted, None, None, None, None, 0.0, kcluster_sizes,
                   gqa_group)


def svg_ear_value_error_scores_triton(
    *,
    qcentroids: torch.Tensor,
    k_sorted: torch.Tensor,
    v_sorted: torch.Tensor,
    kcentroids: torch.Tensor,
    vcentroids: torch.Tensor,
    kcluster_sizes: torch.Tensor,
    gqa_group: int,
    var_k_diag: torch.Tensor | None = None,
    jensen_var_cap: float = 0.0,
    block_q: int = 16,
    block_n: int = 32,
    num_warps: int = 4,
    num_stages: int = 1,
    logical_tokens: int | None = None,
) -> torch.Tensor:
    """Log value-error (Equation-8) routing scores [QH, Qc, Kc] (svg_ear.py:453-531)."""
    if not qcentroids.is_cuda:
        raise RuntimeError("svg_ear_value_error_scores_triton requires CUDA tensors.")
    q_heads, q_clusters, dim = qcentroids.shape
    kv_heads, stored_tokens, k_dim = k_sorted.shape
    tokens = stored_tokens if logical_tokens is None else int(logical_tokens)
    k_clusters = kcentroids.shape[1]
    if dim != 128 or k_dim != dim:
        raise RuntimeError(f"SVG-EAR routing requires DIM=128, got q={dim}, k={k_dim}.")
    if q_heads != kv_heads * gqa_group:
        raise RuntimeError(
            f"SVG-EAR routing GQA mismatch: q_heads={q_heads}, kv_heads={kv_heads}, group={gqa_group}."
        )
    if tokens <= 0 or tokens > stored_tokens:
        raise RuntimeError(f"SVG-EAR logical token count {tokens} must be in [1,{stored_tokens}].")
    _check_tiling(block_q, block_n, num_warps, num_stages, "SVG-EAR routing")
    use_jensen = jensen_var_cap > 0.0
    if use_jensen:
        if var_k_diag is None:
            raise RuntimeError("Jensen-aware SVG-EAR routing requires var_k_diag.")
        if var_k_diag.shape != (kv_heads, k_clusters, dim):
            raise RuntimeError(
                "SVG-EAR routing variance shape mismatch: "
                f"got {tuple(var_k_diag.shape)}, expected {(kv_heads, k_clusters, dim)}."
            )
    return _launch(MODE_VALUE_ERROR, qcentroids, k_sorted, v_sorted, kcentroids, vcentroids,
                   var_k_diag if use_jensen else None, float(jensen_var_cap) if use_jensen else 0.0,
                   kcluster_sizes, gqa_group)


def svg_ear_grouped_value_error_scores_triton(
    *,
    qcentroids: torch.Tensor,
    k_sorted: torch.Tensor,
    v_sorted: torch.Tensor,
    kcentroids: torch.Tensor,
    vcentroids: torch.Tensor,
    kcluster_sizes: torch.Tensor,
    gqa_group: int,
    block_q: int = 16,
    block_n: int = 32,
    num_warps: int = 8,
    num_stages: int = 1,
) -> torch.Tensor:
    """Per-Q-head value-error scores with one K/V walk per GQA group (svg_ear.py:534-600).

    The HIP kernel computes every query head of a group against the same K/V
    rows; the scores equal svg_ear_value_error_scores_triton with the same
    gqa_group."""
    if not qcentroids.is_cuda:
        raise RuntimeError("Grouped SVG-EAR routing requires CUDA tensors.")
    q_heads, q_clusters, dim = qcentroids.shape
    kv_heads, tokens, k_dim = k_sorted.shape
    if dim != 128 or k_dim != dim:
        raise RuntimeError(f"Grouped SVG-EAR requires D=128, got q={dim}, k={k_dim}.")
    if q_heads != kv_heads * gqa_group or gqa_group not in {1, 2, 4, 8}:
        raise RuntimeError(
            f"Grouped SVG-EAR head mismatch q={q_heads}, kv={kv_heads}, G={gqa_group}."
        )
    if block_q not in {8, 16} or block_n not in {16, 32, 64}:
        raise RuntimeError("Grouped SVG-EAR supports BQ={8,16}, BN={16,32,64}.")
    if num_warps not in {4, 8} or num_stages not in {1, 2, 3}:
        raise RuntimeError("Grouped SVG-EAR supports warps={4,8}, stages={1,2,3}.")
    return _launch(MODE_VALUE_ERROR, qcentroids, k_sorted, v_sorted, kcentroids, vcentroids, None, 0.0,
                   kcluster_sizes, gqa_group)


def svg_ear_compensation_triton(*, q_flat: torch.Tensor, sparse_flat: torch.Tensor, lse_flat: torch.Tensor,
                                qlabels_gen: torch.Tensor, dynamic_map_query: torch.Tensor,
                                kcentroids: torch.Tensor, kcluster_sizes: torch.Tensor, vcentroids: torch.Tensor,
                                reformulation: str = "skipped", block_q: int = 64, block_k: int = 32) -> torch.Tensor:
    """The sparse output extended by the centroid approximation of the unselected key
    clusters (svg_ear.py:289-369 kernel, :603-678 wrapper; the same checks and error texts).
    Returns fp32 [BH, T, 128].  block_q is ignored (one tiling of 64 rows); block_k, the
    cluster block of the running max, may be 16 or 32."""
    del block_q
    if not q_flat.is_cuda:
        raise RuntimeError("svg_ear_compensation_triton requires CUDA tensors.")
    if reformulation not in {"skipped", "n3_residual"}:
        raise RuntimeError(
            f"SVG-EAR compensation reformulation must be 'skipped' or 'n3_residual', got {reformulation!r}."
        )
    bh, tokens, dim = q_flat.shape
    clusters = kcentroids.shape[1]
    if dim != 128:
        raise RuntimeError(f"SVG-EAR compensation requires DIM=128, got {dim}.")
    if sparse_flat.shape != (bh, tokens, dim):
        raise RuntimeError(
            f"SVG-EAR sparse output shape mismatch: got {tuple(sparse_flat.shape)}, expected {(bh, tokens, dim)}."
        )
    if lse_flat.shape != (bh, tokens):
        raise RuntimeError(f"SVG-EAR LSE shape mismatch: got {tuple(lse_flat.shape)}, expected {(bh, tokens)}.")
    if qlabels_gen.shape != (bh, tokens):
        raise RuntimeError(
            f"SVG-EAR query-label shape mismatch: got {tuple(qlabels_gen.shape)}, expected {(bh, tokens)}."
        )
    if dynamic_map_query.ndim != 3 or dynamic_map_query.shape[0] != bh:
        raise RuntimeError(
            f"SVG-EAR dynamic-map shape mismatch: got {tuple(dynamic_map_query.shape)}, "
            f"expected batch-head dimension {bh}."
        )
    if dynamic_map_query.shape[2] != clusters + 1:
        raise RuntimeError(
            f"SVG-EAR dynamic-map K-cluster mismatch: got {dynamic_map_query.shape[2]}, expected {clusters + 1}."
        )
    expected_stats = (bh, clusters, dim)
    if kcentroids.shape != expected_stats or vcentroids.shape != expected_stats:
        raise RuntimeError(
            f"SVG-EAR centroid shape mismatch: K={tuple(kcentroids.shape)}, "
            f"V={tuple(vcentroids.shape)}, expected={expected_stats}."
        )
    if kcluster_sizes.shape != (bh, clusters):
        raise RuntimeError(
            f"SVG-EAR cluster-size shape mismatch: got {tuple(kcluster_sizes.shape)}, expected {(bh, clusters)}."
        )
    if block_k not in {16, 32}:
        raise NotImplementedError(f"SVG-EAR compensation on the MI355X kernel takes block_k 16 or 32, got {block_k}.")
    dev = _lib.require_gpu(q_flat, sparse_flat, lse_flat, qlabels_gen, dynamic_map_query, kcentroids, kcluster_sizes,
                           vcentroids, what="SVG-EAR compensation")
    qc = q_flat.contiguous() if q_flat.dtype in (torch.bfloat16, torch.float32) else q_flat.float().contiguous()
    sc = (sparse_flat.contiguous() if sparse_flat.dtype in (torch.bfloat16, torch.float32)
          else sparse_flat.float().contiguous())
    lse = lse_flat.float().contiguous()
    labels = qlabels_gen.to(torch.int32).contiguous()
    dmap = (dynamic_map_query != 0).to(torch.uint8).contiguous()
    kc = kcentroids.float().contiguous()
    vc = vcentroids.float().contiguous()
    counts = kcluster_sizes.float().contiguous()
    out = torch.empty((bh, tokens, dim), device=dev, dtype=torch.float32)
    _lib.call("spr_svg_ear_compensation", _lib.ptr(qc), _lib.DTYPE_CODE[qc.dtype], _lib.ptr(sc),
              _lib.DTYPE_CODE[sc.dtype], _lib.ptr(lse), _lib.ptr(labels), _lib.ptr(dmap), int(dmap.shape[1]),
              _lib.ptr(kc), _lib.ptr(counts), _lib.ptr(vc), bh, tokens, dim, clusters,
              1 if reformulation == "n3_residual" else 0, int(block_k), _lib.ptr(out), _lib.stream(dev))
    return out
