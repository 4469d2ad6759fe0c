"""CPU oracle for the SparsePR sparse-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (sparsepr_amd/) imports,
links or calls this module; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, as the checker.

This is a numpy restatement of the reference's semantics (the reference itself
is never imported).  Every function cites the reference file:line it follows.
Order-sensitive pieces (top-p map, exact-FP32 role step, budget selector) live
in the C part, oracle/c/spr_oracle.c, loaded through ctypes below.

Precision conventions (shared with the HIP kernels, see the project design notes):
  * bf16 values are carried as float32 arrays whose values are bf16-representable
    (round-to-nearest-even, `to_bf16`).
  * k-means cross terms are evaluated in float64 (the bf16 products are exact);
    the GPU's fp32 accumulation may flip labels only between near-tied centroids.
  * centroid sums are accumulated in float64 (exact for bf16 inputs), then
    mean32 = float32(sum / count), then (for bf16 centroids) rounded to bf16.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_C_LIB: ctypes.CDLL | None = None


def c_lib() -> ctypes.CDLL:
    """Load oracle/liboracle_c.so (built by oracle/Makefile)."""
    global _C_LIB
    if _C_LIB is None:
        path = _HERE / "liboracle_c.so"
        if not path.exists():
            raise RuntimeError(f"oracle C library missing: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(str(path))
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        i64 = ctypes.c_int64
        i32 = ctypes.c_int32
        lib.spr_oracle_expf.restype = ctypes.c_float
        lib.spr_oracle_expf.argtypes = [ctypes.c_float]
        lib.spr_oracle_expf_array.restype = None
        lib.spr_oracle_expf_array.argtypes = [f32p, f32p, i64]
        lib.oracle_topp_map.restype = None
        lib.oracle_topp_map.argtypes = [
            f32p, f32p, i32p, i64, i32, i32, i32, ctypes.c_float, ctypes.c_float, i32, i32,
            u8p, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.oracle_select_budget.restype = None
        lib.oracle_select_budget.argtypes = [f32p, i32p, i32p, i64, i32, i32, i32, u8p]
        lib.oracle_role_step64.restype = None
        lib.oracle_role_step64.argtypes = [
            f32p, f32p, i64, i64, i32, i32p, f32p, i32p, ctypes.c_void_p,
        ]
        _C_LIB = lib
    return _C_LIB


# ----------------------------------------------------------------------------
# dtype helpers
# ----------------------------------------------------------------------------

def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest-even); result kept as float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(a)
    out = r.view(np.float32).copy()
    out[nan] = np.float32("nan")
    return out


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float32 values."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def expf(x: np.ndarray) -> np.ndarray:
    """Canonical fp32 exp shared with the GPU kernels (oracle/c/spr_oracle.c)."""
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty_like(a)
    c_lib().spr_oracle_expf_array(a, out, a.size)
    return out.reshape(np.shape(x))


# ----------------------------------------------------------------------------
# k-means (flash_kmeans + kmeans_utils)
# ----------------------------------------------------------------------------

def x_sq_for(x: np.ndarray, mode: str) -> np.ndarray:
    """Per-point squared norm as the reference feeds it to the assign kernel.

    mode "bf16": flash_kmeans computes ``(x ** 2).sum(-1)`` into an ``x.dtype``
      buffer (kmeans_triton_impl.py:84-87): bf16(x_i^2) summed, rounded to bf16.
    mode "fp32": the inline-x_sq kernel sums fp32 squares of the bf16 tile
      (kmeans_utils.py:812-814).
    Sums here are float64 (exact), then rounded once.
    """
    x64 = x.astype(np.float64)
    if mode == "bf16":
        sq = to_bf16((x64 * x64).astype(np.float32)).astype(np.float64)
        return to_bf16(sq.sum(-1).astype(np.float32))
    if mode == "fp32":
        return (x64 * x64).sum(-1).astype(np.float32)
    raise ValueError(mode)


def kmeans_assign(x: np.ndarray, c: np.ndarray, x_sq: np.ndarray):
    """Nearest centroid, lowest index among exact minima.

    Follows assign_euclid_triton.py:803-917 (_euclid_assign_kernel):
    dist = x_sq + c_sq - 2 x.c, clamped at 0; c_sq in fp32 from the centroids
    (assign_euclid_triton.py:1282-1283); running argmin with strict `<` across
    tiles and first index within a tile == lowest index overall.
    Returns (labels int32 [B,N], dist float64 [B,N,K]).
    """
    x64 = x.astype(np.float64)
    c64 = c.astype(np.float64)
    c_sq = (c64 * c64).sum(-1).astype(np.float32).astype(np.float64)
    cross = np.matmul(x64, np.swapaxes(c64, 1, 2))
    dist = x_sq.astype(np.float64)[:, :, None] + c_sq[:, None, :] - 2.0 * cross
    dist = np.maximum(dist, 0.0)
    labels = np.argmin(dist, axis=-1).astype(np.int32)  # numpy returns the first minimum
    return labels, dist


def kmeans_assign_tf32(x: np.ndarray, c: np.ndarray, x_sq: np.ndarray | None = None):
    """The flash-kmeans assign on fp32 inputs (assign_euclid_triton.py:863-917,
    kmeans_utils.py:806-834): tl.dot rounds both fp32 operands to TF32 (nearest, ties
    away), so cross = tf32(x) . tf32(c) with exact products (float64 sum here);
    x_sq = fp32 sum of the fp32 squares of x (inline, kmeans_utils.py:812-814) unless
    given; c_sq = fp32 sum of the fp32 squares of c ((centroids.float() ** 2).sum(-1));
    dist = max(x_sq + c_sq - 2 cross, 0), lowest index among exact minima.
    Returns (labels int32 [B, N], dist float64 [B, N, K], x_sq float32 [B, N])."""
    x32 = np.ascontiguousarray(x, np.float32)
    c32 = np.ascontiguousarray(c, np.float32)
    if x_sq is None:
        x_sq = (x32 * x32).astype(np.float64).sum(-1).astype(np.float32)
    c_sq = (c32 * c32).astype(np.float64).sum(-1).astype(np.float32)
    cross = np.matmul(tf32_rna(x32).astype(np.float64), np.swapaxes(tf32_rna(c32).astype(np.float64), 1, 2))
    dist = np.maximum(x_sq.astype(np.float64)[:, :, None] + c_sq.astype(np.float64)[:, None, :] - 2.0 * cross, 0.0)
    return np.argmin(dist, axis=-1).astype(np.int32), dist, x_sq


def label_mismatches_are_ties(labels_gpu, labels_ref, dist, x_sq, c, rel_tol):
    """True if every label disagreement is between centroids whose exact
    distances differ by at most rel_tol * (x_sq + c_sq) (the scale at which the
    fp32 distance is formed)."""
    bad = labels_gpu != labels_ref
    if not bad.any():
        return True, 0
    b_idx, n_idx = np.nonzero(bad)
    c64 = c.astype(np.float64)
    c_sq = (c64 * c64).sum(-1)
    dg = dist[b_idx, n_idx, labels_gpu[b_idx, n_idx]]
    dr = dist[b_idx, n_idx, labels_ref[b_idx, n_idx]]
    scale = x_sq[b_idx, n_idx].astype(np.float64) + np.maximum(
        c_sq[b_idx, labels_gpu[b_idx, n_idx]], c_sq[b_idx, labels_ref[b_idx, n_idx]]
    )
    ok = np.abs(dg - dr) <= rel_tol * np.maximum(scale, 1e-30)
    return bool(ok.all()), int(bad.sum())


def _group_sums(x2: np.ndarray, labels1: np.ndarray, k: int) -> np.ndarray:
    """Per-group float64 column sums of x2 [N, D] (exact for bf16-valued data)."""
    lab = labels1.astype(np.int64)
    x64 = x2.astype(np.float64)
    return np.stack([np.bincount(lab, weights=x64[:, d], minlength=k) for d in range(x64.shape[1])], axis=1)


def centroid_update(x: np.ndarray, labels: np.ndarray, old: np.ndarray, out_bf16: bool):
    """Cluster means; empty clusters keep the old centroid.

    Follows centroid_update_triton.py:316-386 (sums/max(cnt,1), where(cnt==0, old),
    cast to x.dtype) and torch_fallback.py:72-108.  Sums in float64.
    Returns (centroids [B,K,D] float32 (bf16-rounded if out_bf16), mean32, counts int32).
    """
    B, N, D = x.shape
    K = old.shape[1]
    sums = np.zeros((B, K, D), np.float64)
    counts = np.zeros((B, K), np.int64)
    for b in range(B):
        sums[b] = _group_sums(x[b], labels[b], K)
        counts[b] = np.bincount(labels[b], minlength=K)
    mean32 = (sums / np.maximum(counts, 1)[:, :, None]).astype(np.float32)
    mean32 = np.where(counts[:, :, None] == 0, old.astype(np.float32), mean32)
    cent = to_bf16(mean32) if out_bf16 else mean32
    return cent, mean32, counts.astype(np.int32)


def loop_centroid_update(x, labels, old):
    """Double-loop restatement (torch_fallback.py:54-70) used to pin
    centroid_update: per cluster, mean of member rows in float64."""
    B, N, D = x.shape
    K = old.shape[1]
    out = np.zeros((B, K, D), np.float64)
    for b in range(B):
        for k in range(K):
            mask = labels[b] == k
            if mask.any():
                out[b, k] = x[b][mask].astype(np.float64).mean(axis=0)
            else:
                out[b, k] = old[b, k]
    return out


def batch_kmeans_euclid(x, n_clusters, max_iters, tol=0.0, init_centroids=None,
                        x_sq_mode="bf16", out_bf16=True):
    """Lloyd loop with the reference's return convention.

    kmeans_triton_impl.py:102-115: each iteration assigns with the current
    centroids, updates, computes shift = max ||new - old||; breaks *before*
    adopting the update when shift < tol.  Returns labels of the last
    assignment, the adopted centroids, the sizes of the last assignment
    (kmeans_utils.py:1312-1369 also returns sizes) and the iteration count.
    """
    if init_centroids is None:
        raise ValueError("oracle needs explicit initial centroids")
    cent = init_centroids.astype(np.float32)
    x_sq = x_sq_for(x, x_sq_mode)
    labels = counts = None
    it = -1
    for it in range(max_iters):
        labels, _ = kmeans_assign(x, cent, x_sq)
        new, _, counts = centroid_update(x, labels, cent, out_bf16)
        shift = np.sqrt(((new.astype(np.float64) - cent.astype(np.float64)) ** 2).sum(-1)).max()
        if shift < tol:
            break
        cent = new
    return labels, cent, counts, it + 1


def first_k_init(x: np.ndarray, k: int, seed: int) -> np.ndarray:
    """Seeded first-k init used by the synthetic configs: the first k entries of
    a seeded permutation of the N tokens, per batch (same permutation)."""
    rng = np.random.default_rng(seed)
    idx = rng.permutation(x.shape[1])[:k]
    return x[:, idx, :].copy()


def role_step64(features: np.ndarray, centroids: np.ndarray):
    """One exact FP32 D=64 Lloyd step (n8_ops.cu:198-269, role_cluster_step_q64)."""
    f = np.ascontiguousarray(features, np.float32)
    c = np.ascontiguousarray(centroids, np.float32)
    bh, n, d = f.shape
    assert d == 64
    k = c.shape[1]
    labels = np.empty((bh, n), np.int32)
    out = np.empty_like(c)
    sizes = np.empty((bh, k), np.int32)
    best = np.empty((bh, n), np.float32)
    c_lib().oracle_role_step64(f, c, bh, n, k, labels, out, sizes, best.ctypes.data)
    return labels, out, sizes, best


# ----------------------------------------------------------------------------
# permutation
# ----------------------------------------------------------------------------

def argsort_labels(labels: np.ndarray) -> np.ndarray:
    """Stable ascending argsort per row (kmeans_utils.py:1674-1684 uses
    torch.argsort; the within-cluster order is fixed here to ascending token)."""
    return np.argsort(labels, axis=-1, kind="stable").astype(np.int32)


def permute_rows(x: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Y[bh,s] = X[bh, idx[bh,s]] (permute.py:12-43, kmeans_utils.py:1674-1684)."""
    return np.take_along_axis(x, idx[..., None].astype(np.int64), axis=-2)


def inverse_permute_rows(y: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """X[bh, idx[bh,s]] = Y[bh,s] (permute.py:90-119, kmeans_utils.py:1687-1695)."""
    out = np.empty_like(y)
    bh = y.shape[0]
    for h in range(bh):
        out[h, idx[h].astype(np.int64)] = y[h]
    return out


def permute_concat_rows(prefix, suffix, idx):
    """permute(cat(prefix, suffix)) (permute.py:46-87)."""
    return permute_rows(np.concatenate([prefix, suffix], axis=-2), idx)


# ----------------------------------------------------------------------------
# block selection
# ----------------------------------------------------------------------------

def identify_dynamic_map(qc, kc, k_sizes, p, min_kc_ratio=0.0, return_cum=False, bf16=False):
    """Top-p cluster-pair map (kmeans_utils.py:1710-1742), canonical fp32 order.

    qc [BH,Qc,D], kc [BH,Kc,D] float32; k_sizes [BH,Kc] -> bool [BH,Qc,Kc].
    bf16=True follows torch's dtype flow for bfloat16 centroids (bf16 scores,
    bf16 probabilities, bf16 cumsum outputs, threshold compared in bf16).
    """
    qc = np.ascontiguousarray(qc, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    ks = np.ascontiguousarray(k_sizes, np.int32)
    bh, qn, d = qc.shape
    kn = kc.shape[1]
    out = np.zeros((bh, qn, kn), np.uint8)
    preserve = int(min_kc_ratio * kn) if min_kc_ratio > 0 else 0
    cum = np.zeros((bh, qn, kn), np.float32) if return_cum else None
    order = np.zeros((bh, qn, kn), np.int32) if return_cum else None
    c_lib().oracle_topp_map(
        qc, kc, ks, bh, qn, kn, d, np.float32(math.sqrt(d)), np.float32(p), preserve, int(bool(bf16)), out,
        cum.ctypes.data if cum is not None else None,
        order.ctypes.data if order is not None else None,
    )
    if return_cum:
        return out.astype(bool), cum, order
    return out.astype(bool)


def identify_dynamic_map_f64(qc, kc, k_sizes, p, min_kc_ratio=0.0):
    """The same selection evaluated in float64 with numpy's own ops; used to
    pin the canonical fp32 version away from the threshold."""
    bh, qn, d = qc.shape
    kn = kc.shape[1]
    s = np.einsum("bqd,bkd->bqk", qc.astype(np.float64), kc.astype(np.float64)) / math.sqrt(d)
    s = s - s.max(-1, keepdims=True)
    we = k_sizes.astype(np.float64)[:, None, :] * np.exp(s)
    prob = we / np.maximum(we.sum(-1, keepdims=True), 1e-12)
    order = np.argsort(-prob, axis=-1, kind="stable")
    sp = np.take_along_axis(prob, order, -1)
    cum = np.cumsum(sp, -1)
    remove = np.zeros_like(cum, dtype=bool)
    remove[..., 1:] = cum[..., :-1] > p
    if min_kc_ratio > 0:
        remove[..., : int(min_kc_ratio * kn)] = False
    out = np.zeros((bh, qn, kn), bool)
    np.put_along_axis(out, order, ~remove, -1)
    return out, cum, order


def svg_top_p_key_budgets(qc, kc, k_sizes, top_p):
    """Per-q-cluster key-token budgets (n8_v6.py:181-230): the sizes of the key clusters
    kept by the top-p rule, summed.  The reference's chain (fp32 bmm / sqrt(d), max
    shift, exp times sizes, divide by the clamped sum, descending sort, cumsum, keep
    rank 0 and every rank whose preceding cumsum <= top_p) is identify_dynamic_map's
    fp32 chain (kmeans_utils.py:1698-1742) with the same keep rule, so it is evaluated
    by that canonical fp32 restatement.  Returns int64 [BH, Qc]."""
    keep = identify_dynamic_map(np.asarray(qc, np.float32), np.asarray(kc, np.float32), k_sizes, top_p)
    return (keep.astype(np.int64) * np.asarray(k_sizes, np.int64)[:, None, :]).sum(2)


def select_budget(scores, sizes, budgets, mode=0):
    """Budget selector; mode 0 = n8_ops.cu:271-322, mode 1 = selector_budget.py:10-54.
    Returns bool [BH, Qc+1, Kc+1] with the reference's header row/column."""
    s = np.ascontiguousarray(scores, np.float32)
    bh, qn, kn = s.shape
    out = np.zeros((bh, qn + 1, kn + 1), np.uint8)
    c_lib().oracle_select_budget(
        s, np.ascontiguousarray(sizes, np.int32), np.ascontiguousarray(budgets, np.int32),
        bh, qn, kn, int(mode), out)
    return out.astype(bool)


def compact_selected_clusters(mask):
    """Ascending kept ids per row + counts (n8_ops.cu:324-355)."""
    m = np.asarray(mask, bool)
    kn = m.shape[-1]
    flat = m.reshape(-1, kn)
    ids = np.zeros(flat.shape, np.int32)
    counts = np.zeros(flat.shape[0], np.int32)
    for r in range(flat.shape[0]):
        sel = np.nonzero(flat[r])[0]
        ids[r, : sel.size] = sel
        counts[r] = sel.size
    return ids.reshape(m.shape), counts.reshape(m.shape[:-1])


def density(dynamic_map, q_sizes, k_sizes):
    """Kept pairs / all pairs per (cfg, head) (kmeans_utils.py:285-303)."""
    block = q_sizes[..., :, None].astype(np.float64) * k_sizes[..., None, :].astype(np.float64)
    return (block * dynamic_map).sum((-2, -1)) / block.sum((-2, -1))


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------

def _cum(sizes):
    return np.concatenate([np.zeros(sizes.shape[:-1] + (1,), np.int64),
                           np.cumsum(sizes.astype(np.int64), -1)], -1)


def block_sparse_attention_loop(q, k, v, dynamic_map, q_sizes, k_sizes):
    """Loop-faithful restatement of dynamic_block_sparse_fwd_torch
    (kmeans_utils.py:1748-1841): per q-block online softmax over kept k-blocks,
    float32 arithmetic, acc / max(l, 1e-12).  q,k,v [B,H,S,D]."""
    B, H, S, D = q.shape
    qn = q_sizes.shape[-1]
    kn = k_sizes.shape[-1]
    qcum, kcum = _cum(q_sizes), _cum(k_sizes)
    out = np.zeros_like(q, dtype=np.float32)
    scale = np.float32(D ** -0.5)
    for b in range(B):
        for h in range(H):
            for i in range(qn):
                q0, q1 = qcum[b, h, i], qcum[b, h, i + 1]
                if q1 == q0:
                    continue
                qb = q[b, h, q0:q1].astype(np.float32)
                m = np.full((q1 - q0, 1), -np.inf, np.float32)
                l = np.zeros((q1 - q0, 1), np.float32)
                acc = np.zeros((q1 - q0, D), np.float32)
                for j in range(kn):
                    if not dynamic_map[b, h, i, j]:
                        continue
                    k0, k1 = kcum[b, h, j], kcum[b, h, j + 1]
                    if k1 == k0:
                        continue
                    kb = k[b, h, k0:k1].astype(np.float32)
                    vb = v[b, h, k0:k1].astype(np.float32)
                    s = (qb @ kb.T) * scale
                    mn = np.maximum(m, s.max(-1, keepdims=True))
                    pij = np.exp(s - mn)
                    a = np.exp(m - mn)
                    l = l * a + pij.sum(-1, keepdims=True)
                    acc = acc * a + pij @ vb
                    m = mn
                out[b, h, q0:q1] = acc / np.maximum(l, 1e-12)
    return out


def block_sparse_attention_dense(q, k, v, dynamic_map, q_sizes, k_sizes, return_lse=False):
    """Closed form in float64: softmax over the kept keys of each query row.
    Row i of q-cluster a attends key j of k-cluster c iff map[a, c].
    Rows with no kept key get 0 (and lse = -inf)."""
    B, H, S, D = q.shape
    out = np.zeros((B, H, S, D), np.float64)
    lse = np.full((B, H, S), -np.inf, np.float64)
    for b in range(B):
        for h in range(H):
            ql = np.repeat(np.arange(q_sizes.shape[-1]), q_sizes[b, h].astype(np.int64))
            kl = np.repeat(np.arange(k_sizes.shape[-1]), k_sizes[b, h].astype(np.int64))
            mask = dynamic_map[b, h][ql][:, kl]
            s = (q[b, h].astype(np.float64) @ k[b, h].astype(np.float64).T) / math.sqrt(D)
            s = np.where(mask, s, -np.inf)
            mx = s.max(-1, keepdims=True)
            has = np.isfinite(mx[:, 0])
            e = np.exp(s - np.where(np.isfinite(mx), mx, 0.0))
            e = np.where(mask, e, 0.0)
            l = e.sum(-1, keepdims=True)
            o = (e @ v[b, h].astype(np.float64)) / np.maximum(l, 1e-300)
            out[b, h] = np.where(has[:, None], o, 0.0)
            lse[b, h] = np.where(has, mx[:, 0] + np.log(np.maximum(l[:, 0], 1e-300)), -np.inf)
    if return_lse:
        return out, lse
    return out


def dense_attention(q, k, v):
    """softmax(q k^T / sqrt(D)) v in float64 (F.scaled_dot_product_attention,
    n8_v6.py:1236-1243).  q [BH,M,D], k/v [BH,S,D]."""
    d = q.shape[-1]
    s = np.einsum("bmd,bsd->bms", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(d)
    s -= s.max(-1, keepdims=True)
    e = np.exp(s)
    return np.einsum("bms,bsd->bmd", e, v.astype(np.float64)) / e.sum(-1, keepdims=True)


# ----------------------------------------------------------------------------
# probes and reduced-rank residual repair (models/cosmos3/residual_repair.py)
# ----------------------------------------------------------------------------

def _probe_distances(features, labels, num_clusters):
    """Per-token squared distance to its fp32 cluster center.

    Centers: float64 sums (exact for bf16-valued features) / size, rounded to
    fp32 (residual_repair.py:162-180 builds fp32 centers with scatter_add).
    Distance: the reference sums the squared differences with torch's reduction
    (residual_repair.py:65, :160-164), whose fp32 order is unspecified; the
    canonical order here is a sequential fp32 sum (separate multiply and add)
    within each group of 8 consecutive dims, then a balanced pairwise tree over
    the groups in index order (dims and groups zero-padded to 8 x a power of
    two; the padding adds exact zeros, so r <= 8 is the plain sequential sum)."""
    bh, n, r = features.shape
    f = features.astype(np.float32)
    sizes = np.zeros((bh, num_clusters), np.int64)
    centers = np.zeros((bh, num_clusters, r), np.float32)
    for h in range(bh):
        sizes[h] = np.bincount(labels[h], minlength=num_clusters)
        s = _group_sums(f[h], labels[h], num_clusters)
        centers[h] = (s / np.maximum(sizes[h], 1)[:, None]).astype(np.float32)
    gathered = np.take_along_axis(centers, labels[..., None].astype(np.int64), 1)
    diff = (f - gathered).astype(np.float32)
    groups = -(-r // 8)
    span = 1 << (groups - 1).bit_length()  # tree width: groups rounded up to a power of two
    padded = np.zeros((bh, n, span * 8), np.float32)  # zero terms add exactly 0.0
    padded[..., :r] = diff
    d = padded.reshape(bh, n, span, 8)
    part = np.zeros((bh, n, span), np.float32)
    for e in range(8):
        col = d[..., e]
        part = (part + (col * col).astype(np.float32)).astype(np.float32)
    while part.shape[-1] > 1:
        part = (part[..., 0::2] + part[..., 1::2]).astype(np.float32)
    dist = part[..., 0]
    return sizes, dist


def _weights_for(selected, labels, sizes, num_clusters):
    bh = selected.shape[0]
    w = np.zeros(selected.shape, np.float32)
    for h in range(bh):
        sl = labels[h][selected[h]]
        sampled = np.bincount(sl, minlength=num_clusters)
        gw = sizes[h].astype(np.float32) / np.maximum(sampled, 1).astype(np.float32)
        wh = gw[sl]
        w[h] = wh / max(np.float32(wh.mean(dtype=np.float64)), np.float32(1e-20))
    return w


def select_role_equal_probes_vectorized(features, labels, num_clusters, rows):
    """residual_repair.py:118-208.  One representative per group (nearest token
    to the group center, lowest token id on exact ties), groups ordered by size
    descending (stable), first `rows`; empty-group slots fall back to token j.
    Requires rows <= num_clusters."""
    bh, n, _ = features.shape
    count = min(max(1, int(rows)), int(n))
    if count > num_clusters:
        raise RuntimeError("vectorized probes require rows <= num_clusters")
    sizes, dist = _probe_distances(features, labels, num_clusters)
    selected = np.zeros((bh, count), np.int64)
    for h in range(bh):
        best_d = np.full(num_clusters, np.inf, np.float32)
        np.minimum.at(best_d, labels[h], dist[h])
        cand = np.where(dist[h] == best_d[labels[h]], np.arange(n), n)
        best_i = np.full(num_clusters, n, np.int64)
        np.minimum.at(best_i, labels[h], cand)
        order = np.argsort(-sizes[h], kind="stable")
        sel = best_i[order][:count]
        sel = np.where(sel < n, sel, np.arange(count))
        selected[h] = sel
    weights = _weights_for(selected, labels, sizes, num_clusters)
    return selected, weights


def select_role_equal_probes(features, labels, num_clusters, rows):
    """residual_repair.py:36-115.  Representative rounds: each round takes the
    nearest remaining token of every non-exhausted group in size order, until
    `rows` probes are chosen.  Works for rows > num_clusters."""
    bh, n, _ = features.shape
    count = min(max(1, int(rows)), int(n))
    sizes, dist = _probe_distances(features, labels, num_clusters)
    selected = np.zeros((bh, count), np.int64)
    for h in range(bh):
        remaining = dist[h].copy()
        order = np.argsort(-sizes[h], kind="stable")
        chosen = []
        while len(chosen) < count:
            best_d = np.full(num_clusters, np.inf, np.float32)
            np.minimum.at(best_d, labels[h], remaining)
            cand = np.where(remaining == best_d[labels[h]], np.arange(n), n)
            best_i = np.full(num_clusters, n, np.int64)
            np.minimum.at(best_i, labels[h], cand)
            c = best_i[order]
            c = c[c < n]
            if c.size == 0:
                break
            take = c[: count - len(chosen)]
            chosen.extend(take.tolist())
            remaining[take] = np.inf
        if len(chosen) != count:
            raise RuntimeError("probe selection under-filled")
        selected[h] = np.array(chosen, np.int64)
    weights = _weights_for(selected, labels, sizes, num_clusters)
    return selected, weights


def select_first_token_largest_groups(labels, num_clusters, rows):
    """residual_repair.py:211-260: first token of each of the largest groups;
    weight = group size normalized to mean 1."""
    bh, n = labels.shape
    count = min(max(1, int(rows)), int(n))
    if count > num_clusters:
        raise RuntimeError("first-token probes require rows <= num_clusters")
    selected = np.zeros((bh, count), np.int64)
    weights = np.zeros((bh, count), np.float32)
    for h in range(bh):
        sizes = np.bincount(labels[h], minlength=num_clusters)
        first = np.full(num_clusters, n, np.int64)
        np.minimum.at(first, labels[h], np.arange(n))
        order = np.argsort(-sizes, kind="stable")
        sel = first[order][:count]
        sel = np.where(sel < n, sel, np.arange(count))
        selected[h] = sel
        ss = sizes[labels[h][sel]].astype(np.float32)
        weights[h] = ss / max(np.float32(ss.mean(dtype=np.float64)), np.float32(1e-20))
    return selected, weights


def top16_seed() -> np.ndarray:
    """The fixed start of the top-16 subspace iteration (rrr_eigensolver.py:71-81): the
    reduced QR factor Q of C[i][j] = cos((i + 1/2)(j + 1) pi / 64), i < 64, j < 16, as
    LAPACK's Householder QR (numpy's, torch's) returns it."""
    rows = np.arange(64, dtype=np.float64)[:, None]
    cols = np.arange(16, dtype=np.float64)[None, :]
    q, _ = np.linalg.qr(np.cos((rows + 0.5) * (cols + 1.0) * (math.pi / 64.0)))
    return q


def newton_schulz_inv_sqrt(gram: np.ndarray, iters: int):
    """The fixed-count Newton-Schulz inverse square root of rrr_eigensolver.py:31-40 and
    :58-66 over a batch of symmetric matrices: scale = max(||G||_F, 1e-20), N = G / scale,
    X0 = I, X <- X (3 I - N X X) / 2.  Returns (X, scale); X ~ N^(-1/2) where converged."""
    r = gram.shape[-1]
    eye = np.eye(r, dtype=gram.dtype)
    scale = np.maximum(np.sqrt((gram * gram).sum(axis=(-2, -1), keepdims=True)), 1e-20)
    normalized = gram / scale
    inv_sqrt = np.broadcast_to(eye, gram.shape).copy()
    for _ in range(iters):
        squared = inv_sqrt @ inv_sqrt
        inv_sqrt = 0.5 * (inv_sqrt @ (3.0 * eye - normalized @ squared))
    return inv_sqrt, scale


def top16_right_basis(values: np.ndarray, power_iters: int = 8, inv_sqrt_iters: int = 6) -> np.ndarray:
    """top16_right_basis_triton (rrr_eigensolver.py:86-128) in float64: A = V V^T for
    V [BH, 64, 128]; from Q0 (top16_seed), `power_iters` steps Y = A Q, Q = Y X / sqrt(s)
    with (X, s) = newton_schulz_inv_sqrt(Y^T Y); then B = V^T Q and the basis
    B X / sqrt(s) with (X, s) = newton_schulz_inv_sqrt(B^T B).  Not the exact eigenbasis:
    its span is that of V^T A^power_iters Q0, and where a Gram is ill-conditioned the
    six Newton-Schulz steps leave it short of orthonormal, as the reference's is."""
    v = np.asarray(values, np.float64)
    if v.shape[1:] != (64, 128):
        raise RuntimeError(f"N8 top-16 kernel requires [BH,64,128], got {tuple(v.shape)}.")
    a = v @ np.swapaxes(v, 1, 2)
    q = np.broadcast_to(top16_seed(), (v.shape[0], 64, 16)).copy()
    for _ in range(power_iters):
        y = a @ q
        inv_sqrt, scale = newton_schulz_inv_sqrt(np.swapaxes(y, 1, 2) @ y, inv_sqrt_iters)
        q = (y @ inv_sqrt) / np.sqrt(scale)
    raw = np.swapaxes(v, 1, 2) @ q
    inv_sqrt, scale = newton_schulz_inv_sqrt(np.swapaxes(raw, 1, 2) @ raw, inv_sqrt_iters)
    return (raw @ inv_sqrt) / np.sqrt(scale)


def fit_reduced_rank_residual(x_fit, y_fit, rank, ridge, weights=None,
                              basis_source="raw_residual", dtype=np.float64,
                              output_basis_backend="full", decomposition_backend="eigh"):
    """Weighted ridge reduced-rank regression (residual_repair.py:263-465).

    Standardize X with weighted mean/std (scale clamped at 1e-5), center Y.
    M < P: dual solve (Xw Xw^T + ridge I) dual = Yw; weight = Xw^T dual.
    M >= P: primal solve (Xw^T Xw + ridge I) W = Xw^T Yw.
    Basis: top-`rank` eigenvectors of the weighted output gram of the raw
    (centered) residual ("raw_residual") or of the fitted values.  With the
    "skinny" route, M < D and decomposition_backend "triton_top16"
    (residual_repair.py:435-451,497-503) it is top16_right_basis of the weighted
    values instead (the reference's GPU N8 repair, n8_v6.py:1310-1320).
    left = W basis.  Returns (x_mean[BH,1,P], x_scale, y_mean[BH,1,D], left[BH,P,r], basis[BH,D,r]).
    """
    x = x_fit.astype(dtype)
    y = y_fit.astype(dtype)
    bh, m, p = x.shape
    if weights is None:
        w = np.ones((bh, m, 1), dtype)
        x_mean = x.mean(1, keepdims=True)
        x_scale = np.maximum(x.std(1, ddof=1, keepdims=True), 1e-5)
        y_mean = y.mean(1, keepdims=True)
    else:
        w = weights.astype(dtype)[:, :, None]
        w_sum = np.maximum(w.sum(1, keepdims=True), 1e-20)
        x_mean = (w * x).sum(1, keepdims=True) / w_sum
        x_var = (w * (x - x_mean) ** 2).sum(1, keepdims=True) / w_sum
        x_scale = np.maximum(np.sqrt(x_var), 1e-5)
        y_mean = (w * y).sum(1, keepdims=True) / w_sum
    xn = (x - x_mean) / x_scale
    yc = y - y_mean
    sw = np.sqrt(w)
    xw = xn * sw
    yw = yc * sw
    eye_p = np.eye(p, dtype=dtype)
    if m < p:
        gram = xw @ np.swapaxes(xw, 1, 2) + ridge * np.eye(m, dtype=dtype)
        dual = np.linalg.solve(gram, yw)
        weight = np.swapaxes(xw, 1, 2) @ dual
    else:
        gram = np.swapaxes(xw, 1, 2) @ xw + ridge * eye_p
        rhs = np.swapaxes(xw, 1, 2) @ yw
        weight = np.linalg.solve(gram, rhs)
    fitted = xn @ weight
    values = yc if basis_source == "raw_residual" else fitted
    if output_basis_backend == "skinny" and m < y.shape[2] and decomposition_backend == "triton_top16":
        if rank != 16:
            raise RuntimeError(f"triton_top16 requires rank=16, got {rank}.")
        basis = top16_right_basis(values * sw)
    else:
        out_gram = np.swapaxes(values, 1, 2) @ (values * w)
        _evals, evecs = np.linalg.eigh(out_gram)
        basis = evecs[:, :, -rank:]
    left = weight @ basis
    return x_mean, x_scale, y_mean, left, basis


def recover_nonfinite_rrr_state(state, previous):
    """Per-head fallback (residual_repair.py:509-587): a head whose state holds
    a non-finite value takes the previous state, or a zero correction
    (mean 0, scale 1, y_mean 0, left 0, basis 0) when there is none."""
    bh = state[0].shape[0]
    rec = np.zeros(bh, bool)
    for t in state:
        rec |= ~np.isfinite(t.reshape(bh, -1)).all(1)
    if previous is None:
        fb = (np.zeros_like(state[0]), np.ones_like(state[1]), np.zeros_like(state[2]),
              np.zeros_like(state[3]), np.zeros_like(state[4]))
    else:
        fb = previous
    sel = tuple(np.where(rec.reshape((bh,) + (1,) * (c.ndim - 1)), o, c) for c, o in zip(state, fb))
    return sel, rec


def repair_apply(base, x_mean, x_scale, y_mean, left, basis, alpha, norm_cap, role=None):
    """out = base + alpha * (((x - mu)/sigma) left basis^T + y_mean), optional norm cap with
    x = base, or x = [base, role] with role features (repair_features "output_role";
    residual_repair.py:95-155 and :10-92 kernels, :600-646 torch: the split prediction sums
    the base and the role coordinates, the cap compares with the base norm).  float64."""
    b = base.astype(np.float64)
    x = b if role is None else np.concatenate((b, np.asarray(role, np.float64)), axis=-1)
    z = (x - x_mean) / x_scale
    corr = (z @ left) @ np.swapaxes(basis, 1, 2) + y_mean
    if norm_cap > 0.0:
        bn = np.linalg.norm(b, axis=2, keepdims=True)
        cn = np.maximum(np.linalg.norm(corr, axis=2, keepdims=True), 1e-20)
        corr = corr * np.minimum(norm_cap * bn / cn, 1.0)
    return b + alpha * corr


def exact_probe_scatter(out, rows, dense_probes):
    """out[bh, rows[bh,m]] = dense[bh,m] (residual_repair.py:257-282)."""
    o = out.copy()
    for h in range(out.shape[0]):
        o[h, rows[h].astype(np.int64)] = dense_probes[h]
    return o


# ----------------------------------------------------------------------------
# SVG-EAR routing scores (src/sparsepr/kernels/triton/svg_ear.py)
# ----------------------------------------------------------------------------

def tf32_rna(x: np.ndarray) -> np.ndarray:
    """float32 -> TF32 (10 stored mantissa bits), nearest with ties away from zero: the
    input rounding of the reference's tl.dot(..., input_precision="tf32")
    (svg_ear.py:63,157).  Returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x1000) & 0xFFFFE000).astype(np.uint32)
    return b.view(np.float32)


def _cluster_runs(sizes_row: np.ndarray, tokens: int):
    """Consecutive token runs of the clusters from token 0 (the reference's offsets =
    [0, cumsum(sizes)], svg_ear.py:416-426), clamped to the stored tokens."""
    s = np.maximum(sizes_row.astype(np.int64), 0)
    ends = np.minimum(np.cumsum(s), tokens)
    starts = np.minimum(np.concatenate(([0], np.cumsum(s)[:-1])), tokens)
    return starts, ends


# ----------------------------------------------------------------------------
# N8 role metrics and factors (models/cosmos3/operator_kmeans.py)
# ----------------------------------------------------------------------------

def role_metric(x, rows=None, sizes=None, center=False, post_scale=1.0):
    """covariance / key_metric_from_queries / value_metric_from_values (operator_kmeans.py:62-92,
    :491-498) on the sampled rows, and query_metric_from_key_centroids (:517-531) with
    sizes (rows with size <= 0 are left out of the mean and the count) and post_scale 1/d.
    out [BH, D, D] = post_scale / max(count, 1) * sum (x - mean)(x - mean)^T, float64."""
    x = np.asarray(x, np.float64)
    bh, n, d = x.shape
    out = np.zeros((bh, d, d), np.float64)
    for h in range(bh):
        xs = x[h] if rows is None else x[h, np.asarray(rows, np.int64)]
        if sizes is not None:
            xs = xs[np.asarray(sizes[h]) > 0]
        cnt = max(xs.shape[0], 1)
        if center and xs.shape[0] > 0:
            xs = xs - xs.sum(0) / cnt
        out[h] = xs.T @ xs / cnt * post_scale
    return out


def metric_factor(metric, rank):
    """operator_kmeans.py:95-151: eigh of 0.5 (M + M^T), the top `rank` eigenpairs (ascending),
    eigenvalues clamped at 0, factor = V sqrt(lambda / max(mean lambda, 1e-12)).  float64."""
    m = np.asarray(metric, np.float64)
    m = 0.5 * (m + np.swapaxes(m, 1, 2))
    w, v = np.linalg.eigh(m)
    w = np.maximum(w[:, -rank:], 0.0)
    v = v[:, :, -rank:]
    norm = np.maximum(w.mean(1, keepdims=True), 1e-12)
    return v * np.sqrt(w / norm)[:, None, :]


def _cholesky_or_none(a):
    try:
        return np.linalg.cholesky(a)
    except np.linalg.LinAlgError:
        return None


def _cholesky_qr(x, ridge):
    """operator_kmeans.py:326-358 for one head: normalise the columns (norm clamped at 1e-12),
    Gram + max(mean diag, 1e-12) * ridge I, lower Cholesky (identity on failure),
    x L^-T.  Returns (basis, failed)."""
    xn = x / np.maximum(np.linalg.norm(x, axis=0, keepdims=True), 1e-12)
    g = xn.T @ xn
    g = 0.5 * (g + g.T)
    g = g + np.eye(g.shape[0]) * max(float(np.diag(g).mean()), 1e-12) * ridge
    l = _cholesky_or_none(g)
    if l is None:
        return xn, True
    return np.linalg.solve(l, xn.T).T, False


def householder_qr(x):
    """torch.linalg.qr(x, mode="reduced") (operator_kmeans.py:366,371,419): LAPACK geqrf +
    orgqr, i.e. Householder reflections H_k = I - tau_k v_k v_k^T with v_k[k] = 1 and the
    diagonal of R equal to -sign(alpha_k) |x_k| (alpha_k the pivot entry; tau_k = 0 when the
    column below the pivot is zero).  numpy's qr is the same LAPACK pair."""
    q, _ = np.linalg.qr(np.asarray(x, np.float64), mode="reduced")
    return q


def warm_subspace_metric_factor(metric, previous, rank, power_iters=2, orthogonalization="each_cholesky_qr2",
                                ritz_mode="rayleigh_cholesky", rayleigh_ridge=1e-4, cholesky_qr_ridge=1e-5):
    """operator_kmeans.py:219-477 restated in float64: the Householder-QR (each_qr, final_qr)
    and Cholesky-QR orthogonalisations, and the full / rayleigh_cholesky / diagonal /
    previous_scale finishes.  previous [BH, D, r] is the previous basis.  Returns
    (factor, basis, recovered bool [BH]).  The full finish's columns follow eigh's ascending
    eigenvalue order; their signs are eigh's (arbitrary), so only F F^T is defined."""
    m_all = np.asarray(metric, np.float64)
    prev_all = np.asarray(previous, np.float64)
    bh = m_all.shape[0]
    factors, bases, rec = [], [], np.zeros(bh, bool)
    for h in range(bh):
        m, prev = m_all[h], prev_all[h]
        prev_scales = np.maximum(np.linalg.norm(prev, axis=0), 1e-12)
        basis = householder_qr(prev) if orthogonalization == "each_qr" else prev / prev_scales
        diag = None
        failed = False
        for it in range(power_iters):
            applied = m @ basis
            if ritz_mode == "diagonal" and it == power_iters - 1:
                diag = (basis * applied).sum(0)
            if orthogonalization == "each_qr":
                basis = householder_qr(applied)
                continue
            if orthogonalization in ("cholesky_qr", "final_qr"):
                basis = applied / np.maximum(np.linalg.norm(applied, axis=0), 1e-12)
                continue
            basis, f = _cholesky_qr(applied, cholesky_qr_ridge)
            failed |= f
            if orthogonalization == "each_cholesky_qr2" and it == power_iters - 1:
                basis, f = _cholesky_qr(basis, max(cholesky_qr_ridge, 1e-5))
                failed |= f
        if orthogonalization == "final_qr":
            basis = householder_qr(basis)
        elif orthogonalization == "cholesky_qr":
            basis, f = _cholesky_qr(basis, 1e-6)
            failed |= f
        if ritz_mode == "previous_scale":
            factor = basis * prev_scales
        elif ritz_mode == "diagonal":
            ev = np.maximum(diag, 0.0)
            factor = basis * np.sqrt(ev / max(ev.mean(), 1e-12))
        elif ritz_mode == "full":
            ray = basis.T @ (m @ basis)
            ray = 0.5 * (ray + ray.T)
            ev, rot = np.linalg.eigh(ray)
            ev = np.maximum(ev, 0.0)
            factor = (basis @ rot) * np.sqrt(ev / max(ev.mean(), 1e-12))
        else:
            ray = basis.T @ (m @ basis)
            ray = 0.5 * (ray + ray.T)
            norm = max(float(np.diag(ray).mean()), 1e-12)
            l = _cholesky_or_none(ray + np.eye(rank) * norm * rayleigh_ridge)
            if l is None:
                l = _cholesky_or_none(ray + np.eye(rank) * norm * max(1e-2, rayleigh_ridge))
            if l is None:
                l = np.eye(rank)
                failed = True
            factor = basis @ l / np.sqrt(norm)
        failed |= not (np.isfinite(factor).all() and np.isfinite(basis).all())
        factors.append(factor)
        bases.append(basis)
        rec[h] = failed
    return np.stack(factors), np.stack(bases), rec


def project_rows(x, factor, div=None, tf32=False, row_rms=False, eps=1e-6, precision=None, weight=1.0):
    """project_tokens (operator_kmeans.py:534-538), optionally / a per-head divisor (the
    compiled K-centroid projection, n8_v6.py:152-178, whose "high" precision rounds both fp32
    operands to TF32, "medium" to bf16) times weight (the V half of
    _role_kv_init_projection_fp32, :118-126) and normalize_rows_rms (:548-555).  float64
    products."""
    x = np.asarray(x, np.float32)
    f = np.asarray(factor, np.float32)
    prec = precision if precision is not None else ("high" if tf32 else "highest")
    x, f = matmul_precision_operand(x, prec), matmul_precision_operand(f, prec)
    p = np.matmul(x.astype(np.float64), f.astype(np.float64))
    if div is not None:
        p = p / np.asarray(div, np.float64).reshape(-1, 1, 1)
    if row_rms:
        p = p / np.maximum(np.sqrt((p * p).mean(-1, keepdims=True)), eps)
    return weight * p


def svg_ear_value_error_scores(qc, k_sorted, v_sorted, kc, vc, sizes, group, var_k_diag=None,
                               jensen_var_cap=0.0):
    """Log value-error routing scores (svg_ear.py:95-192 kernel, :453-531 wrapper).

    For query centroid q (fp32) and the tokens t of key cluster c:
      l_c = (q . kc) / sqrt(D) [+ 0.5 min(sum_d q_d^2 var_d / D, cap)]      (:133-140)
      l_t = (tf32(q) . k_t) / sqrt(D)                                         (:157)
      m = max(l_c, max_t l_t); w_c = e^(l_c - m); w_t = e^(l_t - m)
      E = sum_t max(w_c^2 |vc|^2 + w_t^2 |v_t|^2 - 2 w_t w_c (v_t . vc), 0)   (:175-182)
      score = log(max(E / n_c, 1e-30)) + 2 m, -inf for an empty cluster      (:186-188)
    The reference keeps m as a running max over BLOCK_N-token chunks and rescales E by
    alpha^2 and w_c by alpha; that is the same quantity in exact arithmetic, so this
    restatement uses the final max directly, in float64.  Query head h reads kv head
    h // group.  Shapes: qc [QH, Qc, D]; k_sorted, v_sorted [KVH, T, D]; kc, vc, var_k_diag
    [KVH, Kc, D]; sizes [KVH, Kc] -> [QH, Qc, Kc] float32."""
    qh_n, qn, d = qc.shape
    kn = kc.shape[1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    out = np.full((qh_n, qn, kn), -np.inf, dtype=np.float64)
    for h in range(qh_n):
        kh = h // group
        q64 = qc[h].astype(np.float64)
        qt = tf32_rna(qc[h]).astype(np.float64)
        starts, ends = _cluster_runs(sizes[kh], k_sorted.shape[1])
        for c in range(kn):
            n = int(ends[c] - starts[c])
            if n <= 0:
                continue
            kcv = kc[kh, c].astype(np.float64)
            vcv = vc[kh, c].astype(np.float64)
            lc = (q64 @ kcv) * scale
            if jensen_var_cap > 0.0:
                s2 = ((q64 * q64) @ var_k_diag[kh, c].astype(np.float64)) / d
                lc = lc + 0.5 * np.minimum(s2, jensen_var_cap)
            kt = k_sorted[kh, starts[c]:ends[c]].astype(np.float64)
            vt = v_sorted[kh, starts[c]:ends[c]].astype(np.float64)
            lt = (qt @ kt.T) * scale
            m = np.maximum(lc, lt.max(axis=1))
            cw = np.exp(lc - m)[:, None]
            tw = np.exp(lt - m[:, None])
            err = cw * cw * (vcv @ vcv) + tw * tw * (vt * vt).sum(axis=1)[None, :] \
                - 2.0 * tw * cw * (vt @ vcv)[None, :]
            e = np.maximum(err, 0.0).sum(axis=1)
            out[h, :, c] = np.log(np.maximum(e / n, 1e-30)) + 2.0 * m
    return out.astype(np.float32)


def svg_ear_compensation(q, sparse, lse, qlabels, dmap, kc, counts, vc, reformulation="skipped", block_k=32):
    """SVG-EAR compensation (svg_ear.py:289-369 kernel, :603-678 wrapper) in float64.

    Starting from the sparse output (numerator sparse, denominator 1, running max lse), the
    key clusters are walked in blocks of block_k: logits l_c = (tf32(q) . tf32(kc_c)) /
    sqrt(D) + log(max(n_c, 1)); a cluster is valid when n_c > 0 and selected when
    dmap[qlabel + 1, c + 1] != 0.  "skipped" adds e^(l_c - M) tf32-weighted V centroids of
    the valid unselected clusters; "n3_residual" adds those of every valid cluster and
    subtracts the selected ones.  Per block the running max M is updated and the state
    rescaled by e^(M_old - M_new) (NaN where both are -inf, as the reference's exp gives).
    out = acc / max(denom, 1e-30).  q [BH, T, D]; sparse [BH, T, D]; lse, qlabels [BH, T];
    dmap [BH, Qc + 1, Kc + 1]; kc, vc [BH, Kc, D]; counts [BH, Kc] -> float32 [BH, T, D]."""
    q = np.asarray(q, np.float32)
    bh, t, d = q.shape
    kn = kc.shape[1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    n3 = reformulation == "n3_residual"
    out = np.empty((bh, t, d), np.float64)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for h in range(bh):
            qt = tf32_rna(q[h]).astype(np.float64)
            acc = np.asarray(sparse[h], np.float64).copy()
            denom = np.ones(t)
            row_max = np.asarray(lse[h], np.float64).copy()
            rows = np.asarray(qlabels[h], np.int64) + 1
            for k0 in range(0, kn, block_k):
                k1 = min(k0 + block_k, kn)
                kct = tf32_rna(np.asarray(kc[h, k0:k1], np.float32)).astype(np.float64)
                vct = tf32_rna(np.asarray(vc[h, k0:k1], np.float32)).astype(np.float64)
                cnt = np.asarray(counts[h, k0:k1], np.float64)
                logits = (qt @ kct.T) * scale + np.log(np.maximum(cnt, 1.0))[None, :]
                valid = (cnt > 0.0)[None, :]
                sel = np.asarray(dmap[h], bool)[rows][:, k0 + 1:k1 + 1]
                take = valid if n3 else (~sel & valid)
                block_max = np.where(take, logits, -np.inf).max(axis=1)
                new_max = np.maximum(row_max, block_max)
                old = np.exp(row_max - new_max)
                w = np.where(take, np.exp(logits - new_max[:, None]), 0.0)
                wt = tf32_rna(w.astype(np.float32)).astype(np.float64)
                if n3:
                    ws = np.where(sel & valid, w, 0.0)
                    wst = tf32_rna(ws.astype(np.float32)).astype(np.float64)
                    acc = acc * old[:, None] + wt @ vct - wst @ vct
                    denom = denom * old + w.sum(axis=1) - ws.sum(axis=1)
                else:
                    acc = acc * old[:, None] + wt @ vct
                    denom = denom * old + w.sum(axis=1)
                row_max = new_max
            out[h] = acc / np.maximum(denom, 1e-30)[:, None]
    return out.astype(np.float32)


def role_projection_rms(x, factor):
    """Role-coordinate projection with row RMS normalisation (role_projection.py:16-55
    kernel, :58-103 wrapper): p = x . tf32(F) (x bf16-representable, so exact in TF32),
    out = p / sqrt(max(mean_r p_r^2, 1e-12)).  x [BH, N, D], factor [BH, D, R] -> float32
    [BH, N, R]; float64 inside."""
    p = np.einsum("bnd,bdr->bnr", x.astype(np.float64), tf32_rna(factor).astype(np.float64))
    ms = np.maximum((p * p).mean(axis=2, keepdims=True), 1e-12)
    return (p / np.sqrt(ms)).astype(np.float32)


def matmul_precision_operand(x, precision):
    """An fp32 operand as torch's fp32 matmul under set_float32_matmul_precision sees it
    (n8_v6.py:77-86): "highest" unchanged, "high" rounded to TF32, "medium" rounded to
    bf16 (nearest even).  float32."""
    x = np.asarray(x, np.float32)
    if precision == "high":
        return tf32_rna(x)
    if precision == "medium":
        return to_bf16(x)
    if precision == "highest":
        return x
    raise ValueError(f"unknown precision {precision!r}")


def role_k_projection_normalize(k, factor, precision="high", weight=1.0):
    """_role_k_projection_normalize_fp32 (n8_v6.py:141-149) under role_kv_matmul_precision
    (the V half of _role_kv_projection_normalize_fp32, :91-103, with weight): key = k . F~
    with F~ the factor as the matmul sees it (k is bf16, unchanged by any of the roundings),
    key_scale = max(sqrt(mean over tokens and rank of key^2), 1e-8) per head; returns
    ((weight key) / key_scale float32, key_scale float32 [BH, 1, 1]).  float64 inside."""
    f = matmul_precision_operand(factor, precision)
    p = np.einsum("bnd,bdr->bnr", k.astype(np.float64), f.astype(np.float64))
    scale = np.maximum(np.sqrt((p * p).mean(axis=(1, 2), keepdims=True)), 1e-8)
    return ((weight * p) / scale).astype(np.float32), scale.astype(np.float32)


def role_kv_projection_normalize(k, v, k_factor, v_factor, v_weight, precision="high"):
    """_role_kv_projection_normalize_fp32 (n8_v6.py:91-103): cat(key / key_scale,
    (v_weight value) / value_scale) along the feature axis.  Returns (features, key_scale,
    value_scale)."""
    kf, ks = role_k_projection_normalize(k, k_factor, precision)
    vf, vs = role_k_projection_normalize(v, v_factor, precision, weight=v_weight)
    return np.concatenate((kf, vf), axis=2), ks, vs


def attention_mass_scores(qc, k_sorted, sizes, group):
    """Log attention mass of each key cluster at each query centroid (svg_ear.py:7-92
    kernel, :372-450 wrapper): score = log(max(sum_t e^(l_t - m), 1e-30)) + m with
    l_t = (tf32(q) . k_t) / sqrt(D), m = max_t l_t; -inf for an empty cluster.  float64,
    final max in place of the running one (same value in exact arithmetic)."""
    qh_n, qn, d = qc.shape
    kn = sizes.shape[1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    out = np.full((qh_n, qn, kn), -np.inf, dtype=np.float64)
    for h in range(qh_n):
        kh = h // group
        qt = tf32_rna(qc[h]).astype(np.float64)
        starts, ends = _cluster_runs(sizes[kh], k_sorted.shape[1])
        for c in range(kn):
            if ends[c] <= starts[c]:
                continue
            lt = (qt @ k_sorted[kh, starts[c]:ends[c]].astype(np.float64).T) * scale
            m = lt.max(axis=1)
            out[h, :, c] = np.log(np.maximum(np.exp(lt - m[:, None]).sum(axis=1), 1e-30)) + m
    return out.astype(np.float32)


# ----------------------------------------------------------------------------
# model-edge fusions: Q/K RMSNorm + RoPE + layout (n8_ops.cu:16-187)
# ----------------------------------------------------------------------------

def round_to(x, dtype):
    """Round float64 values to the model dtype ('bf16', 'fp16', 'fp32'; 'fp64' keeps
    them), returned as float64."""
    x = np.asarray(x, np.float64)
    if dtype == "bf16":
        return to_bf16(x.astype(np.float32)).astype(np.float64)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float64)
    if dtype == "fp32":
        return x.astype(np.float32).astype(np.float64)
    return x


def _rms_normalize(x, w, eps, dtype):
    """x / sqrt(mean(x^2) + eps) * w over the last axis, rounded to the model dtype
    (the rounding boundary the reference keeps before RoPE, n8_ops.cu:78-90,158-170)."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return round_to(x * inv * np.asarray(w, np.float64), dtype)


def wan_qkv_norm_rope_layout(q, k, v, q_weight, k_weight, freq_real, freq_imag, heads, eps, dtype="bf16"):
    """wan_qkv_norm_rope_layout_kernel (n8_ops.cu:16-105): q, k, v [B, L, C]; RMSNorm over
    the C channels of a token, rounded; channels (2i, 2i + 1) of each head rotated as
    (x0 fr - x1 fi, x0 fi + x1 fr) with freq_real / freq_imag [L, D / 2]; outputs
    [B, H, L, D].  float64 arithmetic, rounded to dtype at the norm and at the output."""
    b, l, c = q.shape
    d = c // heads
    fr = np.asarray(freq_real, np.float64)[None, :, None, :]
    fi = np.asarray(freq_imag, np.float64)[None, :, None, :]

    def rope(x):
        x = x.reshape(b, l, heads, d // 2, 2)
        x0, x1 = x[..., 0], x[..., 1]
        out = np.stack((x0 * fr - x1 * fi, x0 * fi + x1 * fr), axis=-1).reshape(b, l, heads, d)
        return round_to(out, dtype).transpose(0, 2, 1, 3)

    qo = rope(_rms_normalize(q, q_weight, eps, dtype))
    ko = rope(_rms_normalize(k, k_weight, eps, dtype))
    vo = np.asarray(v, np.float64).reshape(b, l, heads, d).transpose(0, 2, 1, 3)
    return qo, ko, vo


def cosmos25_qkv_norm_rope_bshd(q, k, v, q_weight, k_weight, rope_angles, heads, eps, dtype="bf16"):
    """cosmos25_qkv_norm_rope_bshd_kernel (n8_ops.cu:107-187): q, k, v [B, S, H * D]; RMSNorm
    over each head's D values with fp32 weights [D], rounded; out[d] = x[d] cos(a[s, d]) -
    x[d + D/2] sin(a[s, d]) for d < D/2 and x[d] cos + x[d - D/2] sin above (the rotate-half
    convention); outputs [B, S, H, D].  float64 arithmetic, rounded to dtype twice."""
    b, s_len, c = q.shape
    d = c // heads
    half = d // 2
    ang = np.asarray(rope_angles, np.float64).reshape(s_len, d)[None, :, None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(x, w):
        r = _rms_normalize(np.asarray(x, np.float64).reshape(b, s_len, heads, d), w, eps, dtype)
        partner = np.concatenate((-r[..., half:], r[..., :half]), axis=-1)
        return round_to(r * cos + partner * sin, dtype)

    return rope(q, q_weight), rope(k, k_weight), np.asarray(v, np.float64).reshape(b, s_len, heads, d)


# ----------------------------------------------------------------------------
# the whole layer (SAP top-p route + block-sparse attention + N8 repair)
# ----------------------------------------------------------------------------

@dataclass
class LayerConfig:
    q_clusters: int
    k_clusters: int
    kmeans_iters: int
    top_p: float
    probes: int
    min_kc_ratio: float = 0.0
    repair_rank: int = 16
    repair_ridge: float = 0.1
    repair_alpha: float = 1.0
    repair_norm_cap: float = 0.0
    init_seed: int = 0
    x_sq_mode: str = "bf16"


def sparsepr_layer(q, k, v, cfg: LayerConfig, timings: dict | None = None, bf16=True, attention="loop"):
    """One SparsePR attention layer on the CPU, float path of the oracle.

    Composition (wan22.py:2221-2276 for the route and attention, n8_v6.py:1174-1444
    for the repair, hunyuanvideo.py:160-239 for the ordering):
      1. k-means of Q and K (Lloyd, fixed iterations, first-k init);
      2. top-p cluster-pair map from the centroids;
      3. permute Q/K/V into cluster order, block-sparse attention, inverse permute;
      4. probes = role-equal representatives of the Q clusters (features = Q),
         dense probe attention, RRR fit, apply, exact probe scatter.
    q, k, v [BH, N, D] float32 (bf16-valued when bf16=True).
    """
    import time

    def mark(name, t0):
        if timings is not None:
            timings[name] = timings.get(name, 0.0) + (time.perf_counter() - t0) * 1e3
        return time.perf_counter()

    t = time.perf_counter()
    bh, n, d = q.shape
    qi = first_k_init(q, cfg.q_clusters, cfg.init_seed)
    ki = first_k_init(k, cfg.k_clusters, cfg.init_seed + 1)
    q_labels, q_cent, q_sizes, _ = batch_kmeans_euclid(
        q, cfg.q_clusters, cfg.kmeans_iters, 0.0, qi, cfg.x_sq_mode, bf16)
    k_labels, k_cent, k_sizes, _ = batch_kmeans_euclid(
        k, cfg.k_clusters, cfg.kmeans_iters, 0.0, ki, cfg.x_sq_mode, bf16)
    t = mark("kmeans", t)
    dmap = identify_dynamic_map(q_cent, k_cent, k_sizes, cfg.top_p, cfg.min_kc_ratio, bf16=bf16)
    t = mark("select", t)
    q_idx = argsort_labels(q_labels)
    k_idx = argsort_labels(k_labels)
    qp, kp, vp = permute_rows(q, q_idx), permute_rows(k, k_idx), permute_rows(v, k_idx)
    t = mark("permute", t)
    if attention == "loop":  # dynamic_block_sparse_fwd_torch's block loop
        o = block_sparse_attention_loop(qp[None], kp[None], vp[None], dmap[None],
                                        q_sizes[None], k_sizes[None])[0]
    else:  # the vectorized masked-dense variant of the same result
        o = block_sparse_attention_dense(qp[None], kp[None], vp[None], dmap[None],
                                         q_sizes[None], k_sizes[None])[0].astype(np.float32)
    if bf16:
        o = to_bf16(o)
    t = mark("attention", t)
    base = inverse_permute_rows(o, q_idx)
    t = mark("permute", t)
    rows_sel = min(cfg.probes, n)
    if rows_sel <= cfg.q_clusters:
        rows, weights = select_role_equal_probes_vectorized(q, q_labels, cfg.q_clusters, rows_sel)
    else:
        rows, weights = select_role_equal_probes(q, q_labels, cfg.q_clusters, rows_sel)
    qprobe = np.take_along_axis(q, rows[..., None], 1)
    dense = dense_attention(qprobe, k, v).astype(np.float32)
    xfit = np.take_along_axis(base, rows[..., None], 1).astype(np.float32)
    yfit = dense - xfit
    state = fit_reduced_rank_residual(xfit, yfit, min(cfg.repair_rank, rows.shape[1], d),
                                      cfg.repair_ridge, weights, dtype=np.float32)
    state, _ = recover_nonfinite_rrr_state(state, None)
    corrected = repair_apply(base, *state, cfg.repair_alpha, cfg.repair_norm_cap)
    corrected = corrected.astype(np.float32)
    if bf16:
        corrected = to_bf16(corrected)
        dense_out = to_bf16(dense)
    else:
        dense_out = dense
    out = exact_probe_scatter(corrected, rows, dense_out)
    mark("repair", t)
    return {
        "out": out, "base": base, "q_labels": q_labels, "k_labels": k_labels,
        "q_centroids": q_cent, "k_centroids": k_cent, "q_sizes": q_sizes,
        "k_sizes": k_sizes, "map": dmap, "rows": rows, "weights": weights,
        "dense": dense, "density": density(dmap, q_sizes, k_sizes),
    }


