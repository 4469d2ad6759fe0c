"""Block-sparse attention over cluster-pair blocks and split-key dense probe
attention on the HIP kernels of csrc/spr_attention.hip."""

from __future__ import annotations

import math

import torch

from .. import _lib

_PLAN_CACHE: dict = {}


HEAD_DIMS = (16, 32, 64, 128)


def _check_qkv(q, k, v, what):
    """Q/K/V on one GPU, all bfloat16 or all float16, head dim in HEAD_DIMS."""
    dev = _lib.require_gpu(q, k, v, what=what)
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError(f"{what}: bfloat16 or float16 Q/K/V of one dtype required, got "
                           f"{q.dtype}/{k.dtype}/{v.dtype}")
    if q.shape[-1] not in HEAD_DIMS:
        raise RuntimeError(f"{what}: head dim {q.shape[-1]} not supported {HEAD_DIMS}")
    return dev


def plan_block_sparse(block_mask_map: torch.Tensor, block_row_sz: torch.Tensor, block_col_sz: torch.Tensor,
                      seq_len: int) -> torch.Tensor:
    """Kept-segment plan for [BHkv, Qc, Kc] maps (one small kernel)."""
    dev = _lib.require_gpu(block_mask_map, what="block-sparse plan")
    bh_kv, qn, kn = block_mask_map.shape
    m = block_mask_map.to(torch.bool).contiguous()
    qs = block_row_sz.to(device=dev, dtype=torch.int32).reshape(bh_kv, qn).contiguous()
    ks = block_col_sz.to(device=dev, dtype=torch.int32).reshape(bh_kv, kn).contiguous()
    nbytes = _lib.query("spr_block_sparse_attention_workspace", bh_kv, qn, kn)
    plan = _lib.workspace(nbytes, dev)
    _lib.call("spr_block_sparse_attention_plan", _lib.ptr(m), _lib.ptr(qs), _lib.ptr(ks), bh_kv, seq_len, qn, kn,
              _lib.ptr(plan), plan.numel(), _lib.stream(dev))
    plan.spr_plan_sizes = (int(bh_kv), int(qn), int(kn), int(seq_len))
    return plan


def plan_block_sparse_from_schedule(selected_ids: torch.Tensor, selected_counts: torch.Tensor,
                                    block_row_sz: torch.Tensor, block_col_sz: torch.Tensor,
                                    seq_len: int) -> torch.Tensor:
    """The kept-segment plan from a selector schedule (svg_ear_select_budget_schedule /
    compact_selected_clusters, n8_ops.cu:573-638): ids int32 [BHkv, Qc, Kc] whose first
    counts[r] entries per row are the kept k-clusters, ascending; counts [BHkv, Qc].  The
    plan equals plan_block_sparse of the equivalent map."""
    dev = _lib.require_gpu(selected_ids, selected_counts, what="block-sparse plan from a schedule")
    if selected_ids.ndim != 3:
        raise RuntimeError(f"selected_ids must be [BHkv, Qc, Kc], got {tuple(selected_ids.shape)}")
    bh_kv, qn, kn = selected_ids.shape
    if tuple(selected_counts.shape) != (bh_kv, qn):
        raise RuntimeError(f"selected_counts must be {(bh_kv, qn)}, got {tuple(selected_counts.shape)}")
    ids = selected_ids.to(torch.int32).contiguous()
    counts = selected_counts.to(torch.int32).contiguous()
    qs = block_row_sz.to(device=dev, dtype=torch.int32).reshape(bh_kv, qn).contiguous()
    ks = block_col_sz.to(device=dev, dtype=torch.int32).reshape(bh_kv, kn).contiguous()
    nbytes = _lib.query("spr_block_sparse_attention_workspace", bh_kv, qn, kn)
    plan = _lib.workspace(nbytes, dev)
    _lib.call("spr_block_sparse_attention_plan_schedule", _lib.ptr(ids), _lib.ptr(counts), _lib.ptr(qs), _lib.ptr(ks),
              bh_kv, seq_len, qn, kn, _lib.ptr(plan), plan.numel(), _lib.stream(dev))
    plan.spr_plan_sizes = (int(bh_kv), int(qn), int(kn), int(seq_len))
    return plan


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_mask_map: torch.Tensor,
                           block_row_sz: torch.Tensor, block_col_sz: torch.Tensor, *, return_lse: bool = False,
                           plan: torch.Tensor | None = None, scale: float | None = None,
                           q_index: torch.Tensor | None = None, k_index: torch.Tensor | None = None):
    """q [BHq, S, D], k/v [BHkv, S, D] bf16 or fp16 cluster-contiguous, D in (16, 32, 64,
    128); map [BHkv, Qc, Kc]; sizes [BHkv, Qc] / [BHkv, Kc].  Returns out [BHq, S, D] in
    the input dtype (and lse [BHq, S]).

    With q_index int32 [BHq, S] (the stable argsort of the query labels), q and
    the outputs stay in token order: cluster-sorted row r is token q_index[r].
    With k_index int32 [BHkv, S] (the stable argsort of the key labels), k and v
    stay in token order: cluster-sorted key position p is token k_index[p]."""
    dev = _check_qkv(q, k, v, "block-sparse attention")
    bh_q, s, d = q.shape
    bh_kv = k.shape[0]
    if k.shape != (bh_kv, s, d) or v.shape != k.shape:
        raise RuntimeError(f"K/V shape {tuple(k.shape)} / {tuple(v.shape)} does not match Q {tuple(q.shape)}")
    if bh_q % bh_kv != 0:
        raise RuntimeError(f"Q heads ({bh_q}) must be divisible by KV heads ({bh_kv})")
    _, qn, kn = block_mask_map.shape
    if plan is None:
        plan = plan_block_sparse(block_mask_map.to(dev), block_row_sz, block_col_sz, s)
    # a plan from plan_block_sparse* carries the sizes it was built for (the kernels check
    # them too, and write NaN over the output when they differ)
    built = getattr(plan, "spr_plan_sizes", None)
    if built is not None and built != (int(bh_kv), int(qn), int(kn), int(s)):
        raise RuntimeError(f"block-sparse attention: the plan was built for (bh_kv, qn, kn, seq_len) = {built}, "
                           f"not {(int(bh_kv), int(qn), int(kn), int(s))}")
    need = int(_lib.query("spr_block_sparse_attention_workspace", bh_kv, qn, kn))
    if plan.numel() < need or plan.device != dev:
        raise RuntimeError(f"block-sparse attention: the plan ({plan.numel()} bytes on {plan.device}) was not built "
                           f"for bh_kv={bh_kv}, qn={qn}, kn={kn} ({need} bytes on {dev})")
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    qi = None
    if q_index is not None:
        if tuple(q_index.shape) != (bh_q, s):
            raise RuntimeError(f"q_index must have shape {(bh_q, s)}, got {tuple(q_index.shape)}")
        qi = q_index.to(device=dev, dtype=torch.int32).contiguous()
    ki = None
    if k_index is not None:
        if tuple(k_index.shape) != (bh_kv, s):
            raise RuntimeError(f"k_index must have shape {(bh_kv, s)}, got {tuple(k_index.shape)}")
        ki = k_index.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty_like(qc)
    lse = torch.empty((bh_q, s), dtype=torch.float32, device=dev) if return_lse else None
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(d)
    _lib.call("spr_block_sparse_attention_run_ex", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(plan),
              plan.numel(), bh_q, bh_kv, s, d, qn, kn, sc, _lib.DTYPE_CODE[qc.dtype], _lib.ptr(qi), _lib.ptr(ki),
              _lib.ptr(out), _lib.ptr(lse), _lib.stream(dev))
    return (out, lse) if return_lse else out


def cached_plan(key, token, block_mask_map, block_row_sz, block_col_sz, seq_len):
    """Plan cache keyed by an owner key; a matching token reuses the plan
    (kmeans_utils.py:2229-2267 semantics)."""
    entry = _PLAN_CACHE.get(key)
    shape = (tuple(block_mask_map.shape), int(seq_len))
    if entry is not None and entry[0] == token and entry[1] == shape:
        return entry[2]
    plan = plan_block_sparse(block_mask_map, block_row_sz, block_col_sz, seq_len)
    _PLAN_CACHE[key] = (token, shape, plan)
    return plan


def clear_plan_cache():
    _PLAN_CACHE.clear()


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float | None = None,
                    out_dtype: torch.dtype = torch.float32, return_lse: bool = False, nsplit: int | None = None):
    """softmax(q k^T * scale) v for few query rows: q [BHq, M, D], k/v [BHkv, S, D]
    bf16 or fp16 -> [BHq, M, D] in out_dtype (fp32, bf16 or fp16)."""
    dev = _check_qkv(q, k, v, "dense attention")
    bh_q, m, d = q.shape
    bh_kv, s_kv, _ = k.shape
    if v.shape != k.shape or k.shape[2] != d:
        raise RuntimeError("dense attention: K/V shape mismatch")
    if bh_q % bh_kv != 0:
        raise RuntimeError("dense attention: Q heads must be a multiple of KV heads")
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise RuntimeError("dense attention: out_dtype must be float32, bfloat16 or float16")
    if nsplit is None:
        # one round of workgroups, two per CU over the chip's 256 CUs (measured at the
        # C4 shape: 21 splits 0.31 ms, 42 splits 0.32 ms, 43 splits 0.36 ms, since a
        # workgroup past a whole round leaves a nearly empty last one)
        mtiles = max(1, (m + 127) // 128)
        nsplit = max(1, min(512 // (bh_q * mtiles), s_kv // 512))
    qc = q.contiguous()
    # K/V whose rows are packed within each head, with one head stride for both (a slice
    # of the keys of a larger tensor), are read in place
    in_place = (k.stride(2) == 1 and k.stride(1) == d and v.stride() == k.stride() and k.stride(0) >= s_kv * d
                and k.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0)
    kc, vc = (k, v) if in_place else (k.contiguous(), v.contiguous())
    out = torch.empty((bh_q, m, d), dtype=out_dtype, device=dev)
    lse = torch.empty((bh_q, m), dtype=torch.float32, device=dev) if return_lse else None
    ws = _lib.workspace(_lib.query("spr_dense_attention_workspace", bh_q, m, d, nsplit), dev)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(d)
    _lib.call("spr_dense_attention_strided_ex", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), bh_q, bh_kv, m, s_kv,
              kc.stride(0) if bh_kv > 1 else s_kv * d, d, sc, _lib.DTYPE_CODE[qc.dtype], nsplit, _lib.ptr(out),
              _lib.DTYPE_CODE[out_dtype], _lib.ptr(lse), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
    return (out, lse) if return_lse else out
