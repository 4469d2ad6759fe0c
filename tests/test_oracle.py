"""Pins the CPU oracle against the reference's known-answer test, closed forms,
brute force on tiny inputs and invariants.  CPU only."""

import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


# --------------------------------------------------------------------------- exp

def test_expf_within_two_ulp_of_float64_exp(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.uniform(-87.0, 0.0, 200000), rng.uniform(-1.0, 1.0, 50000),
        rng.uniform(0.0, 88.0, 20000), np.array([0.0, -0.0, -1e-30, -86.99, -87.0, 1.0])
    ]).astype(np.float32)
    got = oracle.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(got, ref).max() <= 2
    assert oracle.expf(np.array([-87.5, -200.0], np.float32)).tolist() == [0.0, 0.0]
    assert np.isinf(oracle.expf(np.array([89.0], np.float32))[0])
    # the top of the range, where round(x log2 e) = 128: finite up to ln(FLT_MAX)
    top = np.linspace(88.0, 88.7228, 4001).astype(np.float32)
    got = oracle.expf(top)
    assert np.isfinite(got).all()
    assert _ulp_diff(got, np.exp(top.astype(np.float64)).astype(np.float32)).max() <= 2
    over = np.array([88.7230, 88.8, 88.99], np.float32)  # e^x > FLT_MAX
    assert np.isinf(oracle.expf(over)).all()


def test_bf16_rounding_nearest_even(oracle):
    # 1 + 2^-8 is exactly half way between bf16(1) and bf16(1 + 2^-7): ties to even (1.0)
    vals = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38], np.float32)
    got = oracle.to_bf16(vals)
    assert got[0] == 1.0
    assert got[1] == np.float32(1.0 + 2 ** -6)
    assert got[2] == -2.5
    assert np.isinf(oracle.to_bf16(np.array([3.4e38], np.float32))[0])


# --------------------------------------------------------------------------- selector KAT

def test_selector_known_answer(oracle):
    kat = json.loads((GOLDEN / "selector_kat.json").read_text())
    scores = np.array(kat["scores"], np.float32)
    sizes = np.array(kat["sizes"], np.int32)
    budgets = np.array(kat["budgets"], np.int32)
    for mode in (0, 1):
        out = oracle.select_budget(scores, sizes, budgets, mode=mode)
        assert out[0, 1:, 1:].tolist() == kat["expected_mask"]
        assert out[0, 0, 0] == kat["expected_header_00"]
        assert bool(out[0, 1:, 0].all()) == kat["expected_column0"]
    ids, counts = oracle.compact_selected_clusters(np.array(kat["expected_mask"]))
    assert counts.tolist() == kat["expected_counts"][0]
    assert ids[0, :3].tolist() == kat["expected_ids"][0][0]
    assert ids[1, :2].tolist() == kat["expected_ids"][0][1]


def test_selector_modes_differ_only_on_zero_cost_before_crossing(oracle):
    # sorted costs [5, 0, 3], budget 6: mode 0 adds the first positive crossing (c2);
    # mode 1 adds sorted position `count`=1, the zero-cost cluster c1.
    scores = np.array([[[3.0, 2.0, 1.0]]], np.float32)
    sizes = np.array([[5, 0, 3]], np.int32)
    budgets = np.array([[6]], np.int32)
    m0 = oracle.select_budget(scores, sizes, budgets, 0)[0, 1, 1:]
    m1 = oracle.select_budget(scores, sizes, budgets, 1)[0, 1, 1:]
    assert m0.tolist() == [True, False, True]
    assert m1.tolist() == [True, True, False]


def _select_budget_brute(scores, sizes, budgets):
    """Python restatement of the per-row walk (mode 0) for random cases."""
    bh, qn, kn = scores.shape
    out = np.zeros((bh, qn, kn), bool)
    for h in range(bh):
        for i in range(qn):
            order = sorted(range(kn), key=lambda j: (-float(scores[h, i, j]), j))
            sel, cross = 0, None
            for j in order:
                c = int(sizes[h, j])
                if c <= 0:
                    continue
                if cross is None and sel + c <= budgets[h, i]:
                    out[h, i, j] = True
                    sel += c
                elif cross is None:
                    cross = j
            if budgets[h, i] > 0 and sel < budgets[h, i] and cross is not None:
                out[h, i, cross] = True
    return out


def test_selector_random_vs_walk(oracle):
    rng = np.random.default_rng(3)
    scores = rng.integers(0, 6, (2, 5, 9)).astype(np.float32)  # many ties
    sizes = rng.integers(0, 7, (2, 9)).astype(np.int32)
    budgets = rng.integers(0, 25, (2, 5)).astype(np.int32)
    got = oracle.select_budget(scores, sizes, budgets, 0)[:, 1:, 1:]
    assert (got == _select_budget_brute(scores, sizes, budgets)).all()


# --------------------------------------------------------------------------- k-means

def _bf16_data(oracle, rng, shape, scale=1.0):
    return oracle.to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def test_assign_matches_brute_force_with_planted_ties(oracle):
    rng = np.random.default_rng(1)
    x = _bf16_data(oracle, rng, (2, 40, 8))
    c = _bf16_data(oracle, rng, (2, 6, 8))
    c[:, 4] = c[:, 1]  # duplicate centroid: every tie must resolve to index 1
    x[:, 0] = c[:, 1]  # a point exactly on a centroid
    x_sq = oracle.x_sq_for(x, "fp32")
    labels, _ = oracle.kmeans_assign(x, c, x_sq)
    for b in range(2):
        for n in range(40):
            best, bi = None, None
            for k in range(6):
                dot = sum(float(x[b, n, t]) * float(c[b, k, t]) for t in range(8))
                csq = float(np.float32(sum(float(c[b, k, t]) ** 2 for t in range(8))))
                d = max(float(x_sq[b, n]) + csq - 2.0 * dot, 0.0)
                if best is None or d < best:
                    best, bi = d, k
            assert labels[b, n] == bi
    assert (labels != 4).all()


def test_assign_tf32_brute_force_and_rounding_matters(oracle):
    """kmeans_assign_tf32 against a loop with explicitly TF32-rounded operands, and a planted
    point whose nearest centroid differs between TF32 and exact fp32 products (a dropped
    rounding step fails the second check)."""
    rng = np.random.default_rng(41)
    x = rng.standard_normal((2, 30, 16)).astype(np.float32)
    c = rng.standard_normal((2, 7, 16)).astype(np.float32)
    labels, dist, x_sq = oracle.kmeans_assign_tf32(x, c)
    for b in range(2):
        for n in range(30):
            xs = float(np.float32(sum(float(np.float32(v * v)) for v in x[b, n])))
            best = None
            for k in range(7):
                xt, ct = oracle.tf32_rna(x[b, n]), oracle.tf32_rna(c[b, k])
                cross = sum(float(a) * float(bb) for a, bb in zip(xt, ct))
                cs = float(np.float32(sum(float(np.float32(v * v)) for v in c[b, k])))
                d = max(xs + cs - 2.0 * cross, 0.0)
                if best is None or d < best[0]:
                    best = (d, k)
            assert labels[b, n] == best[1]
    # 1-D case: x = 1 + 1.25 * 2^-10 rounds to 1 + 2^-10 in TF32; centroids 1 and 1 + 2^-9.
    # Exact products put x nearer 1 + 2^-9; with the TF32 cross term both distances equal
    # x_sq - 1 - 2^-9, and the lower index, 0, wins.
    xv = np.zeros((1, 1, 16), np.float32)
    cv = np.zeros((1, 2, 16), np.float32)
    xv[0, 0, 0] = 1 + 1.25 * 2 ** -10
    cv[0, 0, 0], cv[0, 1, 0] = 1.0, 1 + 2 ** -9
    tl, td, _ = oracle.kmeans_assign_tf32(xv, cv)
    exact = ((xv[0, 0, 0].astype(np.float64) - cv[0, :, 0].astype(np.float64)) ** 2)
    assert int(np.argmin(exact)) == 1 and tl[0, 0] == 0


def test_x_sq_modes(oracle):
    rng = np.random.default_rng(2)
    x = _bf16_data(oracle, rng, (1, 16, 128))
    f32 = oracle.x_sq_for(x, "fp32")
    b16 = oracle.x_sq_for(x, "bf16")
    ref = (x.astype(np.float64) ** 2).sum(-1)
    assert np.allclose(f32, ref, rtol=1e-6)
    assert np.allclose(b16, ref, rtol=2 ** -7)
    assert (oracle.to_bf16(b16) == b16).all()


def test_centroid_update_matches_double_loop(oracle):
    rng = np.random.default_rng(4)
    x = _bf16_data(oracle, rng, (2, 64, 16))
    labels = rng.integers(0, 7, (2, 64)).astype(np.int32)
    labels[labels == 5] = 6  # cluster 5 empty
    old = _bf16_data(oracle, rng, (2, 7, 16))
    cent, mean32, counts = oracle.centroid_update(x, labels, old, out_bf16=True)
    loop = oracle.loop_centroid_update(x, labels, old)
    assert (mean32 == loop.astype(np.float32)).all()
    assert (cent == oracle.to_bf16(loop.astype(np.float32))).all()
    assert (cent[:, 5] == old[:, 5]).all()
    assert counts.sum(1).tolist() == [64, 64]


def test_lloyd_return_convention(oracle):
    rng = np.random.default_rng(5)
    x = _bf16_data(oracle, rng, (1, 200, 8))
    init = oracle.first_k_init(x, 5, seed=0)
    # tol larger than any shift: break in the first iteration, return the init
    labels, cent, counts, iters = oracle.batch_kmeans_euclid(x, 5, 7, tol=1e9, init_centroids=init)
    assert iters == 1
    assert (cent == init).all()
    l0, _ = oracle.kmeans_assign(x, init, oracle.x_sq_for(x, "bf16"))
    assert (labels == l0).all()
    # tol = 0 never breaks: labels come from the last assignment, centroids from the last update
    labels, cent, counts, iters = oracle.batch_kmeans_euclid(x, 5, 3, tol=0.0, init_centroids=init)
    assert iters == 3
    c = init
    for _ in range(3):
        lab, _ = oracle.kmeans_assign(x, c, oracle.x_sq_for(x, "bf16"))
        c, _, cnt = oracle.centroid_update(x, lab, c, True)
    assert (lab == labels).all() and (c == cent).all() and (cnt == counts).all()


def test_lloyd_objective_non_increasing(oracle):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, 500, 4)).astype(np.float32)
    c = oracle.first_k_init(x, 8, seed=1)
    prev = None
    for _ in range(6):
        lab, dist = oracle.kmeans_assign(x, c, oracle.x_sq_for(x, "fp32"))
        obj = np.take_along_axis(dist, lab[..., None].astype(np.int64), -1).sum()
        if prev is not None:
            assert obj <= prev * (1 + 1e-6)
        prev = obj
        c, _, _ = oracle.centroid_update(x, lab, c, out_bf16=False)


def test_role_step64_vs_float64(oracle):
    rng = np.random.default_rng(7)
    f = rng.standard_normal((2, 300, 64)).astype(np.float32)
    c = rng.standard_normal((2, 20, 64)).astype(np.float32)
    c[:, 11] = c[:, 3]  # exact tie: lower index wins
    labels, out, sizes, best = oracle.role_step64(f, c)
    d64 = ((f[:, :, None, :].astype(np.float64) - c[:, None, :, :]) ** 2).sum(-1)
    ref = d64.argmin(-1)
    srt = np.sort(d64, -1)
    clear = (srt[..., 1] - srt[..., 0]) > 1e-4 * srt[..., 0]
    assert (labels[clear] == ref[clear]).all()
    assert (labels != 11).all()
    assert np.allclose(best, np.take_along_axis(d64, labels[..., None].astype(np.int64), -1)[..., 0], rtol=1e-5)
    assert sizes.sum(1).tolist() == [300, 300]
    for h in range(2):
        for k in range(20):
            m = labels[h] == k
            exp = f[h][m].astype(np.float64).mean(0).astype(np.float32) if m.any() else c[h, k]
            assert (out[h, k] == exp).all()


# --------------------------------------------------------------------------- permutation

def test_permutation_invariants(oracle):
    rng = np.random.default_rng(8)
    labels = rng.integers(0, 9, (3, 257)).astype(np.int32)
    idx = oracle.argsort_labels(labels)
    sorted_labels = np.take_along_axis(labels, idx.astype(np.int64), -1)
    assert (np.diff(sorted_labels, axis=-1) >= 0).all()
    for h in range(3):
        assert sorted(idx[h].tolist()) == list(range(257))
        for a, b in zip(idx[h][:-1], idx[h][1:]):
            if labels[h, a] == labels[h, b]:
                assert a < b  # stable
    x = rng.standard_normal((3, 257, 5)).astype(np.float32)
    y = oracle.permute_rows(x, idx)
    assert (y[1, 7] == x[1, idx[1, 7]]).all()
    assert (oracle.inverse_permute_rows(y, idx) == x).all()
    pre, suf = x[:, :200], x[:, 200:]
    idx2 = oracle.argsort_labels(labels)
    assert (oracle.permute_concat_rows(pre, suf, idx2) == oracle.permute_rows(x, idx2)).all()


# --------------------------------------------------------------------------- top-p map

def _map_inputs(rng, bh=2, qn=6, kn=11, d=16, empty=(3,)):
    qc = rng.standard_normal((bh, qn, d)).astype(np.float32)
    kc = rng.standard_normal((bh, kn, d)).astype(np.float32)
    ks = rng.integers(1, 50, (bh, kn)).astype(np.int32)
    for e in empty:
        ks[:, e] = 0
    return qc, kc, ks


def test_topp_map_matches_float64_away_from_threshold(oracle):
    rng = np.random.default_rng(9)
    for p in (0.5, 0.8, 0.9, 0.95):
        qc, kc, ks = _map_inputs(rng)
        got, cum32, _ = oracle.identify_dynamic_map(qc, kc, ks, p, return_cum=True)
        ref, cum64, _ = oracle.identify_dynamic_map_f64(qc, kc, ks, p)
        near = (np.abs(cum64 - p) < 1e-5).any(-1)
        assert (got[~near] == ref[~near]).all()
        assert np.allclose(cum32, cum64, atol=1e-6)


def test_topp_map_invariants_and_brute_force(oracle):
    rng = np.random.default_rng(10)
    qc, kc, ks = _map_inputs(rng, bh=1, qn=4, kn=7, d=8, empty=(2,))
    p = 0.7
    got = oracle.identify_dynamic_map(qc, kc, ks, p)
    for i in range(4):
        s = [sum(float(qc[0, i, t]) * float(kc[0, j, t]) for t in range(8)) / math.sqrt(8) for j in range(7)]
        mx = max(s)
        w = [ks[0, j] * math.exp(s[j] - mx) for j in range(7)]
        tot = sum(w)
        probs = [wj / tot for wj in w]
        order = sorted(range(7), key=lambda j: (-probs[j], j))
        keep, cum = set(), 0.0
        for r, j in enumerate(order):
            if r == 0 or cum <= p:
                keep.add(j)
            cum += probs[j]
        assert {j for j in range(7) if got[0, i, j]} == keep
        assert got[0, i].sum() >= 1
        assert not got[0, i, 2] or len(keep) == 7  # empty cluster only kept when everything is
        assert sum(probs[j] for j in keep) >= p - 1e-6
    many = oracle.identify_dynamic_map(qc, kc, ks, 0.01, min_kc_ratio=0.5)
    assert (many.sum(-1) >= 3).all()


# --------------------------------------------------------------------------- attention

def _block_problem(oracle, rng, qn=5, kn=7, d=16, zero_q=2, zero_k=4, empty_row=1):
    qs = rng.integers(1, 9, (1, 2, qn))
    ks = rng.integers(1, 9, (1, 2, kn))
    qs[..., zero_q] = 0
    ks[..., zero_k] = 0
    S = int(max(qs.sum(-1).max(), ks.sum(-1).max()))
    qs[..., -1] += S - qs.sum(-1)
    ks[..., -1] += S - ks.sum(-1)
    q = rng.standard_normal((1, 2, S, d)).astype(np.float32)
    k = rng.standard_normal((1, 2, S, d)).astype(np.float32)
    v = rng.standard_normal((1, 2, S, d)).astype(np.float32)
    m = rng.random((1, 2, qn, kn)) < 0.5
    m[..., empty_row, :] = False
    return q, k, v, m, qs, ks


def test_block_sparse_loop_equals_dense_closed_form(oracle):
    rng = np.random.default_rng(11)
    for _ in range(3):
        q, k, v, m, qs, ks = _block_problem(oracle, rng)
        loop = oracle.block_sparse_attention_loop(q, k, v, m, qs, ks)
        dense, lse = oracle.block_sparse_attention_dense(q, k, v, m, qs, ks, return_lse=True)
        assert np.allclose(loop, dense, atol=2e-5, rtol=1e-4)
        # rows of the all-dropped q-cluster are zero with lse = -inf
        r0 = int(qs[0, 0, :1].sum())
        r1 = r0 + int(qs[0, 0, 1])
        assert (dense[0, 0, r0:r1] == 0).all() and np.isneginf(lse[0, 0, r0:r1]).all()


def test_block_sparse_full_map_is_dense_attention(oracle):
    rng = np.random.default_rng(12)
    q, k, v, m, qs, ks = _block_problem(oracle, rng, empty_row=0, zero_q=0, zero_k=0)
    m[:] = True
    full = oracle.block_sparse_attention_dense(q, k, v, m, qs, ks)
    d = oracle.dense_attention(q[0], k[0], v[0])
    assert np.allclose(full[0], d, atol=1e-12)
    # per-row closed form for one row
    s = q[0, 1, 3].astype(np.float64) @ k[0, 1].T.astype(np.float64) / math.sqrt(q.shape[-1])
    e = np.exp(s - s.max())
    assert np.allclose(d[1, 3], (e / e.sum()) @ v[0, 1].astype(np.float64))


def test_density(oracle):
    m = np.array([[[[True, False], [False, True]]]])
    qs = np.array([[[1, 3]]])
    ks = np.array([[[2, 2]]])
    # kept pairs = 1*2 + 3*2 = 8 of 16
    assert oracle.density(m, qs, ks)[0, 0] == 0.5


# --------------------------------------------------------------------------- probes

def _probe_data(oracle, rng, bh=2, n=120, r=6, c=9):
    f = oracle.to_bf16(rng.standard_normal((bh, n, r)).astype(np.float32))
    labels = rng.integers(0, c, (bh, n)).astype(np.int32)
    labels[:, :3] = 0
    labels[labels == 4] = 5  # group 4 empty
    return f, labels


def test_probe_selection_brute_force(oracle):
    rng = np.random.default_rng(13)
    f, labels = _probe_data(oracle, rng)
    f[0, 10] = f[0, 20]
    labels[0, 10] = labels[0, 20]  # duplicate token: lower id wins
    rows, weights = oracle.select_role_equal_probes_vectorized(f, labels, 9, 6)
    for h in range(2):
        sizes = [int((labels[h] == g).sum()) for g in range(9)]
        order = sorted(range(9), key=lambda g: (-sizes[g], g))
        expect = []
        for g in order[:6]:
            mem = [t for t in range(120) if labels[h, t] == g]
            if not mem:
                expect.append(None)
                continue
            cen = [sum(float(f[h, t, j]) for t in mem) / len(mem) for j in range(6)]
            dist = [sum((float(f[h, t, j]) - cen[j]) ** 2 for j in range(6)) for t in mem]
            best = min(dist)
            expect.append(min(t for t, dd in zip(mem, dist) if dd <= best * (1 + 1e-6) + 1e-12))
        for pos, e in enumerate(expect):
            assert rows[h, pos] == (pos if e is None else e)
        assert abs(weights[h].mean() - 1.0) < 1e-6
        sl = labels[h][rows[h]]
        raw = np.array([sizes[g] / max(1, int((sl == g).sum())) for g in sl])
        assert np.allclose(weights[h], raw / raw.mean(), rtol=1e-6)
    assert rows[0].tolist().count(20) == 0 or 10 not in rows[0].tolist()


@pytest.mark.parametrize("r", [6, 20, 128])
def test_probe_distance_canonical_order(oracle, r):
    """The distance order the kernel reproduces: per token, fp32 sums of squared
    differences over groups of 8 dims in sequence, then a pairwise tree over the groups
    (padded to a power of two).  Checked bit for bit against a scalar float32 loop in that
    order, and against float64 distances to 1e-6 relative."""
    rng = np.random.default_rng(100 + r)
    bh, n, c = 1, 24, 3
    f = oracle.to_bf16(rng.standard_normal((bh, n, r)).astype(np.float32))
    labels = rng.integers(0, c, (bh, n)).astype(np.int32)
    _sizes, got = oracle._probe_distances(f, labels, c)
    f32 = np.float32
    for t in range(n):
        mem = f[0, labels[0] == labels[0, t]].astype(np.float64)
        cen = (mem.sum(0) / len(mem)).astype(np.float32)
        diff = [f32(f32(f[0, t, j]) - cen[j]) for j in range(r)]
        groups = -(-r // 8)
        span = 1
        while span < groups:
            span *= 2
        parts = []
        for g in range(span):
            acc = f32(0.0)
            for e in range(8):
                j = 8 * g + e
                dj = diff[j] if j < r else f32(0.0)
                acc = f32(acc + f32(dj * dj))
            parts.append(acc)
        while len(parts) > 1:
            parts = [f32(parts[2 * u] + parts[2 * u + 1]) for u in range(len(parts) // 2)]
        assert got[0, t] == parts[0]
        exact = float(((f[0, t].astype(np.float64) - mem.mean(0)) ** 2).sum())
        assert abs(float(got[0, t]) - exact) <= 1e-6 * max(exact, 1e-12) + 1e-6 * float(cen.astype(np.float64) @ cen)


def test_probe_loop_equals_vectorized_when_rows_fit(oracle):
    rng = np.random.default_rng(14)
    f, labels = _probe_data(oracle, rng)
    a = oracle.select_role_equal_probes_vectorized(f, labels, 9, 7)
    b = oracle.select_role_equal_probes(f, labels, 9, 7)
    assert (a[0] == b[0]).all() and np.allclose(a[1], b[1])
    # more probes than groups: rounds; every row distinct and valid
    rows, w = oracle.select_role_equal_probes(f, labels, 9, 30)
    for h in range(2):
        assert len(set(rows[h].tolist())) == 30
    first, wf = oracle.select_first_token_largest_groups(labels, 9, 5)
    for h in range(2):
        sizes = [int((labels[h] == g).sum()) for g in range(9)]
        order = sorted(range(9), key=lambda g: (-sizes[g], g))[:5]
        assert first[h].tolist() == [int(np.nonzero(labels[h] == g)[0][0]) for g in order]
        raw = np.array([sizes[g] for g in order], np.float64)
        assert np.allclose(wf[h], raw / raw.mean(), rtol=1e-6)


# --------------------------------------------------------------------------- RRR

def _rrr_inputs(rng, bh=3, m=40, p=12, d=10, weighted=True):
    x = rng.standard_normal((bh, m, p)).astype(np.float32)
    y = (x @ rng.standard_normal((bh, p, d)).astype(np.float32) * 0.3
         + 0.05 * rng.standard_normal((bh, m, d)).astype(np.float32))
    w = rng.uniform(0.5, 2.0, (bh, m)).astype(np.float32) if weighted else None
    return x, y, w


@pytest.mark.parametrize("m,p", [(40, 12), (8, 12)])
def test_rrr_normal_equations_and_basis(oracle, m, p):
    rng = np.random.default_rng(15)
    x, y, w = _rrr_inputs(rng, m=m, p=p)
    rank, ridge = 4, 0.1
    x_mean, x_scale, y_mean, left, basis = oracle.fit_reduced_rank_residual(x, y, rank, ridge, w)
    wt = w.astype(np.float64)[:, :, None]
    assert np.allclose((wt * x).sum(1, keepdims=True) / wt.sum(1, keepdims=True), x_mean)
    xn = (x - x_mean) / x_scale
    assert np.allclose((wt * xn).sum(1), 0, atol=1e-9)
    assert np.allclose((wt * xn ** 2).sum(1) / wt.sum(1), 1, atol=1e-9)
    xw, yw = xn * np.sqrt(wt), (y - y_mean) * np.sqrt(wt)
    # unrestricted ridge solution from the SVD of Xw (a different algorithm)
    u, s, vt = np.linalg.svd(xw, full_matrices=False)
    w_svd = np.swapaxes(vt, 1, 2) @ ((s / (s ** 2 + ridge))[:, :, None] * (np.swapaxes(u, 1, 2) @ yw))
    assert np.allclose(left, w_svd @ basis, atol=1e-8)
    # basis: orthonormal, invariant subspace of the output gram with the top eigenvalues
    g = np.swapaxes(y - y_mean, 1, 2) @ ((y - y_mean) * wt)
    assert np.allclose(np.swapaxes(basis, 1, 2) @ basis, np.eye(rank), atol=1e-9)
    proj = basis @ np.swapaxes(basis, 1, 2)
    assert np.allclose(proj @ g @ basis, g @ basis, atol=1e-8)
    ev = np.linalg.eigvalsh(g)
    assert np.allclose(np.trace(np.swapaxes(basis, 1, 2) @ g @ basis, axis1=1, axis2=2), ev[:, -rank:].sum(1))


def test_rrr_zero_residual_gives_zero_correction(oracle):
    rng = np.random.default_rng(16)
    x, _, w = _rrr_inputs(rng, p=12, d=12)
    y = np.zeros((3, 40, 12), np.float32)
    state = oracle.fit_reduced_rank_residual(x, y, 4, 0.1, w)
    base = rng.standard_normal((3, 50, 12))
    out = oracle.repair_apply(base, *state, 1.0, 0.0)
    assert np.allclose(out, base, atol=1e-12)


def test_recover_nonfinite_rrr_state(oracle):
    rng = np.random.default_rng(17)
    x, y, w = _rrr_inputs(rng)
    state = oracle.fit_reduced_rank_residual(x, y, 4, 0.1, w)
    bad = tuple(t.copy() for t in state)
    bad[3][1, 0, 0] = np.nan
    sel, rec = oracle.recover_nonfinite_rrr_state(bad, None)
    assert rec.tolist() == [False, True, False]
    assert (sel[3][1] == 0).all() and (sel[1][1] == 1).all()
    assert (sel[3][0] == state[3][0]).all()
    sel2, rec2 = oracle.recover_nonfinite_rrr_state(bad, state)
    assert (sel2[3][1] == state[3][1]).all()


def test_repair_norm_cap_and_scatter(oracle):
    rng = np.random.default_rng(18)
    x, y, w = _rrr_inputs(rng, p=12, d=12)
    state = oracle.fit_reduced_rank_residual(x, y, 4, 0.1, w)
    base = rng.standard_normal((3, 30, 12))
    capped = oracle.repair_apply(base, *state, 1.0, 0.05)
    corr = capped - base
    assert (np.linalg.norm(corr, axis=2) <= 0.05 * np.linalg.norm(base, axis=2) + 1e-9).all()
    rows = np.array([[0, 5], [1, 2], [29, 3]])
    dense = rng.standard_normal((3, 2, 12))
    out = oracle.exact_probe_scatter(capped, rows, dense)
    assert (out[2, 29] == dense[2, 0]).all() and (out[0, 1] == capped[0, 1]).all()


@pytest.mark.parametrize("ridge", [0.0, 0.3])
def test_repair_apply_at_fit_rows_satisfies_normal_equations(oracle, ridge):
    """A full-rank fit (rank = D, M > P = D) applied at its own fit rows: the residual
    y - (apply(x) - x) satisfies the weighted ridge normal equations, sum w r = 0 and
    sum w xn^T r = ridge W, with xn standardised here by numpy's weighted average and W the
    map the state applies.  A wrong standardisation or a dropped y_mean in the apply fails."""
    rng = np.random.default_rng(41)
    bh, m, d = 2, 40, 6
    x = (3.0 * rng.standard_normal((bh, m, d)) + rng.uniform(-2, 2, (bh, 1, d))).astype(np.float32)
    y = (x @ rng.standard_normal((bh, d, d)) * 0.2 + 0.3 * rng.standard_normal((bh, m, d))
         + np.array([1.5, -2.0, 0.5, 3.0, -1.0, 0.25])).astype(np.float32)
    w = rng.uniform(0.5, 2.0, (bh, m)).astype(np.float32)
    state = oracle.fit_reduced_rank_residual(x, y, d, ridge, w)
    pred = oracle.repair_apply(x, *state, 1.0, 0.0) - x.astype(np.float64)
    r = y.astype(np.float64) - pred
    for h in range(bh):
        wh = w[h].astype(np.float64)
        mu = np.average(x[h].astype(np.float64), axis=0, weights=wh)
        sd = np.sqrt(np.average((x[h] - mu) ** 2, axis=0, weights=wh))
        xn = (x[h] - mu) / sd
        assert np.abs(wh @ r[h]).max() <= 1e-9 * np.abs(y[h]).sum()
        W = state[3][h] @ state[4][h].T
        assert np.allclose((xn * wh[:, None]).T @ r[h], ridge * W, atol=1e-8)
    # the apply at other rows uses the same affine map (a check of linearity in base)
    b2 = rng.standard_normal((bh, 7, d))
    a0 = oracle.repair_apply(np.zeros((bh, 1, d)), *state, 1.0, 0.0)
    a1 = oracle.repair_apply(b2, *state, 1.0, 0.0)
    assert np.allclose(a1 - b2 - a0, (b2 / state[1]) @ state[3] @ np.swapaxes(state[4], 1, 2), atol=1e-10)


def test_repair_apply_hand_worked(oracle):
    """Two tokens worked out by hand (dyadic numbers, exact), with x_scale != 1, y_mean != 0
    and alpha != 1; then the norm cap on a token whose correction is (6, 8) against a base
    of norm 5."""
    base = np.array([[[1.0, 2.0], [3.0, 5.0]]])
    x_mean = np.array([[[1.0, 1.0]]])
    x_scale = np.array([[[2.0, 4.0]]])
    y_mean = np.array([[[0.5, -1.0]]])
    left = np.array([[[1.0], [2.0]]])
    basis = np.array([[[3.0], [-1.0]]])
    out = oracle.repair_apply(base, x_mean, x_scale, y_mean, left, basis, 0.5, 0.0)
    # token 0: z = (0, 1/4), z.left = 1/2, corr = (3/2, -1/2) + (1/2, -1) = (2, -3/2)
    # token 1: z = (1, 1),   z.left = 3,   corr = (9, -3) + (1/2, -1)   = (19/2, -4)
    assert (out == np.array([[[2.0, 1.25], [7.75, 3.0]]])).all()
    # base (3, 4): z = ((3-1)/2, (4-0)/4) = (1, 1); z.left = 3; corr = (6, 6) + (0, 2) = (6, 8);
    # cap 0.25 * |base| / |corr| = 0.125 -> (0.75, 1); alpha 2 -> (4.5, 6)
    capped = oracle.repair_apply(np.array([[[3.0, 4.0]]]), np.array([[[1.0, 0.0]]]), x_scale,
                                 np.array([[[0.0, 2.0]]]), left, np.array([[[2.0], [2.0]]]), 2.0, 0.25)
    assert np.allclose(capped, [[[4.5, 6.0]]], rtol=0, atol=1e-12)


def test_repair_apply_role_features_hand_worked(oracle):
    """repair_features "output_role": the role features extend the standardised row, and the
    norm cap compares with the base norm only.  One token by hand: base (1, 2), role (5,);
    z = ((1-1)/2, (2-1)/4, (5-3)/2) = (0, 1/4, 1); left (1, 2, -1) -> z.left = -1/2;
    corr = -1/2 (3, -1) + (1/2, -1) = (-1, -1/2); alpha 2 -> (-1, 1).  With cap 0.1: |base| =
    sqrt 5, |corr| = sqrt(5) / 2, factor 0.2 -> corr (-0.2, -0.1), alpha 2 -> (0.6, 1.8)."""
    base = np.array([[[1.0, 2.0]]])
    role = np.array([[[5.0]]])
    x_mean = np.array([[[1.0, 1.0, 3.0]]])
    x_scale = np.array([[[2.0, 4.0, 2.0]]])
    y_mean = np.array([[[0.5, -1.0]]])
    left = np.array([[[1.0], [2.0], [-1.0]]])
    basis = np.array([[[3.0], [-1.0]]])
    out = oracle.repair_apply(base, x_mean, x_scale, y_mean, left, basis, 2.0, 0.0, role=role)
    assert (out == np.array([[[-1.0, 1.0]]])).all()
    capped = oracle.repair_apply(base, x_mean, x_scale, y_mean, left, basis, 2.0, 0.1, role=role)
    assert np.allclose(capped, [[[0.6, 1.8]]], rtol=0, atol=1e-12)


def test_repair_apply_role_at_fit_rows_satisfies_normal_equations(oracle):
    """A full-rank fit on [base, role] features (P = D + R > M: the dual solve) applied at its
    fit rows with the role rows passed separately: the residual satisfies the ridge normal
    equations sum w xn^T r = ridge W over all P standardised features."""
    rng = np.random.default_rng(43)
    bh, m, d, rr, ridge = 2, 10, 6, 8, 0.4
    base = rng.standard_normal((bh, m, d)) * 2.0 + 1.0
    role = rng.standard_normal((bh, m, rr))
    x = np.concatenate((base, role), axis=2).astype(np.float32)
    y = (rng.standard_normal((bh, m, d)) + 0.5).astype(np.float32)
    w = rng.uniform(0.5, 2.0, (bh, m)).astype(np.float32)
    state = oracle.fit_reduced_rank_residual(x, y, d, ridge, w)
    pred = oracle.repair_apply(x[:, :, :d], *state, 1.0, 0.0, role=x[:, :, d:]) - x[:, :, :d].astype(np.float64)
    r = y.astype(np.float64) - pred
    for h in range(bh):
        wh = w[h].astype(np.float64)
        mu = np.average(x[h].astype(np.float64), axis=0, weights=wh)
        xn = (x[h] - mu) / np.sqrt(np.average((x[h] - mu) ** 2, axis=0, weights=wh))
        W = state[3][h] @ state[4][h].T
        assert np.abs(wh @ r[h]).max() <= 1e-9 * np.abs(y[h]).sum()
        assert np.allclose((xn * wh[:, None]).T @ r[h], ridge * W, atol=1e-8)


@pytest.mark.parametrize("m", [40, 8])
def test_rrr_fitted_basis_by_lstsq(oracle, m):
    """basis_source="fitted_residual": the fitted values from numpy's least squares on the
    ridge-augmented system [x_w; sqrt(ridge) I] W = [y_w; 0] (not the oracle's solve); the
    basis spans the top-rank right singular vectors of sqrt(w) * fitted (numpy SVD)."""
    rng = np.random.default_rng(42)
    x, y, w = _rrr_inputs(rng, m=m, p=12, d=10)
    rank, ridge = 3, 0.2
    x_mean, x_scale, y_mean, left, basis = oracle.fit_reduced_rank_residual(
        x, y, rank, ridge, w, basis_source="fitted_residual")
    raw = oracle.fit_reduced_rank_residual(x, y, rank, ridge, w, basis_source="raw_residual")[4]
    for h in range(x.shape[0]):
        wh = w[h].astype(np.float64)
        mu = np.average(x[h].astype(np.float64), axis=0, weights=wh)
        xn = (x[h] - mu) / np.sqrt(np.average((x[h] - mu) ** 2, axis=0, weights=wh))
        ym = np.average(y[h].astype(np.float64), axis=0, weights=wh)
        sw = np.sqrt(wh)[:, None]
        a = np.vstack((xn * sw, math.sqrt(ridge) * np.eye(x.shape[2])))
        rhs = np.vstack(((y[h] - ym) * sw, np.zeros((x.shape[2], y.shape[2]))))
        W = np.linalg.lstsq(a, rhs, rcond=None)[0]
        _, _, vt = np.linalg.svd(sw * (xn @ W))
        want = vt[:rank].T @ vt[:rank]
        assert np.allclose(basis[h] @ basis[h].T, want, atol=1e-8)
        assert not np.allclose(raw[h] @ raw[h].T, want, atol=1e-3)  # the two sources differ here
        assert np.allclose(left[h], W @ basis[h], atol=1e-8)


def test_rrr_unweighted_uses_unbiased_std(oracle):
    """Without weights the scale is the unbiased (ddof 1) standard deviation, clamped at
    1e-5, and the means are plain means; at M = 3 ddof changes the scale by sqrt(3/2)."""
    rng = np.random.default_rng(43)
    x = rng.standard_normal((2, 3, 5)).astype(np.float32)
    x[1, :, 4] = 7.0  # a constant feature: std 0 -> the clamp
    y = rng.standard_normal((2, 3, 4)).astype(np.float32)
    x_mean, x_scale, y_mean, _, _ = oracle.fit_reduced_rank_residual(x, y, 2, 0.1, None)
    assert np.allclose(x_mean[:, 0], x.astype(np.float64).mean(1))
    assert np.allclose(y_mean[:, 0], y.astype(np.float64).mean(1))
    want = np.maximum(np.std(x.astype(np.float64), axis=1, ddof=1), 1e-5)
    assert np.allclose(x_scale[:, 0], want, rtol=1e-12)
    assert x_scale[1, 0, 4] == 1e-5


# --------------------------------------------------------------------------- top-16 subspace

TOP16_SEED_SIGNS = [-1, -1, -1, -1, -1, 1, 1, 1, 1, -1, -1, -1, 1, 1, 1, -1]


def test_top16_seed_is_signed_dct(oracle):
    """The seed's columns are DCT-II vectors (orthogonal, norm sqrt(32)), so LAPACK's
    Householder QR returns them scaled by 1/sqrt(32) and the signs of R's diagonal; numpy
    and torch (the reference calls torch.linalg.qr) agree on those signs."""
    import torch

    q = oracle.top16_seed()
    i = np.arange(64)[:, None]
    j = np.arange(16)[None, :]
    c = np.cos((i + 0.5) * (j + 1) * math.pi / 64)
    assert np.allclose(c.T @ c, 32 * np.eye(16), atol=1e-12)
    assert np.allclose(q, c / math.sqrt(32) * np.array(TOP16_SEED_SIGNS), atol=1e-14)
    ct = torch.cos((torch.arange(64.0)[:, None] + 0.5) * (torch.arange(16.0)[None, :] + 1.0) * (math.pi / 64.0))
    _, r = torch.linalg.qr(ct, mode="reduced")
    assert torch.sign(torch.diagonal(r)).tolist() == TOP16_SEED_SIGNS


def test_newton_schulz_matches_spectral_route(oracle):
    """The matrix Newton-Schulz iteration equals the scalar recurrence x <- x (3 - v x^2) / 2
    (x0 = 1) applied to the eigenvalues v of G / ||G||_F (numpy eigh): a transposed product,
    a wrong constant or a different normalisation fails; converged, X = (G / s)^(-1/2)."""
    rng = np.random.default_rng(44)
    a = rng.standard_normal((3, 30, 16)) * np.exp(-0.3 * np.arange(16))
    g = np.swapaxes(a, 1, 2) @ a
    for iters in (1, 2, 6):
        x, s = oracle.newton_schulz_inv_sqrt(g, iters)
        lam, e = np.linalg.eigh(g)
        v = lam / np.linalg.norm(g, axis=(1, 2))[:, None]
        f = np.ones_like(v)
        for _ in range(iters):
            f = 0.5 * f * (3.0 - v * f * f)
        want = e @ (f[:, :, None] * np.swapaxes(e, 1, 2))
        assert np.allclose(x, want, atol=1e-9 * np.abs(want).max())
        assert np.allclose(s[:, 0, 0], np.sqrt((g ** 2).sum((1, 2))))
    # a well-conditioned Gram converges in a dozen steps (the uncoupled iteration lets
    # rounding errors grow again over many more steps once converged)
    a = rng.standard_normal((3, 200, 16))
    g = np.swapaxes(a, 1, 2) @ a
    x, s = oracle.newton_schulz_inv_sqrt(g, 12)
    assert np.allclose(x @ (g / s) @ x, np.eye(16), atol=1e-10)


def test_top16_basis_span_and_convergence(oracle):
    """The basis spans V^T (V V^T)^k Q0 (a QR of that product, another route), for k = 8 and
    k = 3; with many iterations on a spectrum with a gap at 16 it converges to the exact top-16
    right singular subspace (numpy SVD), orthonormal."""
    rng = np.random.default_rng(45)
    u, _ = np.linalg.qr(rng.standard_normal((2, 64, 64)))
    vt, _ = np.linalg.qr(rng.standard_normal((2, 128, 64)))
    s = np.concatenate((np.linspace(3.0, 2.0, 16), np.linspace(1.0, 0.1, 48)))
    v = (u * s) @ np.swapaxes(vt, 1, 2)
    q0 = oracle.top16_seed()
    for k in (8, 3):
        # the default is the reference's 8 power iterations
        b = oracle.top16_right_basis(v) if k == 8 else oracle.top16_right_basis(v, power_iters=k)
        a = v @ np.swapaxes(v, 1, 2)
        direct = np.swapaxes(v, 1, 2) @ np.linalg.matrix_power(a, k) @ q0
        qd, _ = np.linalg.qr(direct)
        qb, _ = np.linalg.qr(b)
        assert np.allclose(qb @ np.swapaxes(qb, 1, 2), qd @ np.swapaxes(qd, 1, 2), atol=1e-9)
    b = oracle.top16_right_basis(v, power_iters=60, inv_sqrt_iters=12)
    exact = vt[:, :, :16]
    assert np.allclose(b @ np.swapaxes(b, 1, 2), exact @ np.swapaxes(exact, 1, 2), atol=1e-8)
    assert np.allclose(np.swapaxes(b, 1, 2) @ b, np.eye(16), atol=1e-8)


def test_top16_fit_is_the_skinny_triton_route(oracle):
    """The fit with output_basis_backend "skinny", M < D and "triton_top16" uses the top-16
    basis of the weighted values (raw residual or weighted fitted values), and left = W basis;
    other routes keep the exact eigenbasis; rank other than 16 is refused as the reference does."""
    rng = np.random.default_rng(46)
    x = rng.standard_normal((2, 64, 128)).astype(np.float32)
    y = (rng.standard_normal((2, 64, 64)) * np.exp(-0.1 * np.arange(64))) @ rng.standard_normal((2, 64, 128)) / 20
    w = rng.uniform(0.5, 2.0, (2, 64)).astype(np.float32)
    for source in ("raw_residual", "fitted_residual"):
        st = oracle.fit_reduced_rank_residual(x, y, 16, 0.1, w, basis_source=source, output_basis_backend="skinny",
                                              decomposition_backend="triton_top16")
        ex = oracle.fit_reduced_rank_residual(x, y, 16, 0.1, w, basis_source=source, output_basis_backend="skinny")
        sw = np.sqrt(w.astype(np.float64))[:, :, None]
        yc = (y - st[2]) * sw
        xw = (x - st[0]) / st[1] * sw
        dual = np.linalg.solve(xw @ np.swapaxes(xw, 1, 2) + 0.1 * np.eye(64), yc)
        vals = yc if source == "raw_residual" else yc - 0.1 * dual  # sqrt(w) fitted = y_w - ridge dual
        assert np.allclose(st[4], oracle.top16_right_basis(vals), atol=1e-10)
        assert np.allclose(st[3], np.swapaxes(xw, 1, 2) @ dual @ st[4], atol=1e-8)
        assert not np.allclose(st[4] @ np.swapaxes(st[4], 1, 2), ex[4] @ np.swapaxes(ex[4], 1, 2), atol=1e-3)
        full =oracle.fit_reduced_rank_residual(x, y, 16, 0.1, w, basis_source=source,
                                                decomposition_backend="triton_top16")
        assert np.allclose(full[4] @ np.swapaxes(full[4], 1, 2), ex[4] @ np.swapaxes(ex[4], 1, 2), atol=1e-8)
    with pytest.raises(RuntimeError, match="rank=16"):
        oracle.fit_reduced_rank_residual(x, y, 8, 0.1, w, output_basis_backend="skinny",
                                         decomposition_backend="triton_top16")


# --------------------------------------------------------------------------- whole layer

def test_layer_runs_and_probe_rows_are_exact(oracle):
    rng = np.random.default_rng(19)
    bh, n, d = 2, 256, 16
    q = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    k = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    cfg = oracle.LayerConfig(q_clusters=8, k_clusters=16, kmeans_iters=3, top_p=0.9, probes=8)
    res = oracle.sparsepr_layer(q, k, v, cfg)
    out = res["out"]
    assert out.shape == (bh, n, d) and np.isfinite(out).all()
    for h in range(bh):
        assert (out[h, res["rows"][h]] == oracle.to_bf16(res["dense"][h])).all()
    assert ((res["density"] > 0) & (res["density"] <= 1)).all()


def _torch_identify_dynamic_map(qc, kc, k_sizes, p, min_kc_ratio=0.0):
    """The reference's op sequence (kmeans_utils.py:1698-1742) run with torch on
    the CPU in the centroids' own dtype: an independent implementation of the
    dtype flow (torch's matmul, rounding, sort and cumsum)."""
    import torch

    D = qc.shape[-1]
    kc_num = kc.shape[-2]
    s = torch.matmul(qc, kc.transpose(-2, -1)) / (D ** 0.5)
    w = k_sizes.unsqueeze(-2).float()
    input_dtype = s.dtype
    sf = s.float()
    e = torch.exp(sf - sf.max(-1, keepdim=True)[0])
    we = w * e
    probs = (we / we.sum(-1, keepdim=True).clamp(min=1e-12)).to(input_dtype)
    sp, si = torch.sort(probs, dim=-1, descending=True, stable=True)
    cum = torch.cumsum(sp, dim=-1)
    rem = cum > p
    rem[..., 1:] = rem[..., :-1].clone()
    rem[..., 0] = False
    if min_kc_ratio > 0:
        rem[..., : int(min_kc_ratio * kc_num)] = False
    out = torch.zeros(probs.shape, dtype=torch.bool)
    out.scatter_(-1, si, ~rem)
    return out, cum.float()


@pytest.mark.parametrize("bf16", [False, True])
def test_topp_map_matches_torch_dtype_flow(oracle, bf16):
    import torch

    rng = np.random.default_rng(21 + bf16)
    for p in (0.8, 0.9):
        qc = (0.4 * rng.standard_normal((3, 16, 64))).astype(np.float32)
        kc = (0.4 * rng.standard_normal((3, 40, 64))).astype(np.float32)
        ks = rng.integers(0, 300, (3, 40)).astype(np.int32)
        if bf16:
            qc, kc = oracle.to_bf16(qc), oracle.to_bf16(kc)
        dt = torch.bfloat16 if bf16 else torch.float32
        ref, cum = _torch_identify_dynamic_map(torch.from_numpy(qc).to(dt), torch.from_numpy(kc).to(dt),
                                               torch.from_numpy(ks), p)
        got, gcum, gorder = oracle.identify_dynamic_map(qc, kc, ks, p, bf16=bf16, return_cum=True)
        ref = ref.numpy()
        cum = cum.numpy()
        # Every row whose kept set differs is counted and must be a tie at its decisive
        # ranks: the two chains' cumulative masses there lie within one unit of the last
        # place (bf16: 2^-8 below 1; fp32: a few ulps of the summation order) of p.
        tol = 2.0 ** -8 if bf16 else 4 * 2.0 ** -24
        bad = np.nonzero((got != ref).any(-1))
        for h, i in zip(*bad):
            co, ct = int(got[h, i].sum()), int(ref[h, i].sum())
            lo, hi = min(co, ct), max(co, ct)
            assert lo != hi, f"row {(h, i)}: same count, different clusters"
            # ranks lo-1 .. hi-2 decide (cumsum <= p keeps the next rank)
            for r in range(lo - 1, hi - 1):
                assert abs(float(gcum[h, i, r]) - p) <= tol and abs(float(cum[h, i, r]) - p) <= tol, (
                    f"row {(h, i)} rank {r}: oracle cum {gcum[h, i, r]}, torch cum {cum[h, i, r]}, p {p}")
        assert len(bad[0]) <= max(2, got.shape[0] * got.shape[1] // 10), f"{len(bad[0])} tie rows"


# --------------------------------------------------------------------------- SVG-EAR routing scores

def test_tf32_rounding_ties_away_from_zero(oracle):
    # 1 + 2^-11 lies half way between TF32 neighbours 1 and 1 + 2^-10: ties away from zero
    # (round-to-nearest-even would give 1)
    vals = np.array([1 + 2 ** -11, 1 + 2 ** -12, -(1 + 2 ** -11), 1 + 3 * 2 ** -12, 1 + 2 ** -10, 3.0],
                    np.float32)
    got = oracle.tf32_rna(vals)
    assert got.tolist() == [1 + 2 ** -10, 1.0, -(1 + 2 ** -10), 1 + 2 ** -10, 1 + 2 ** -10, 3.0]
    x = np.random.default_rng(1).standard_normal(100000).astype(np.float32)
    t = oracle.tf32_rna(x)
    assert (t.view(np.uint32) & 0x1FFF == 0).all()
    # within half a TF32 ulp
    ulp = np.ldexp(1.0, np.frexp(np.abs(x).astype(np.float64))[1] - 11)
    assert (np.abs(t.astype(np.float64) - x) <= ulp / 2).all()


def _svg_case(rng, qh, group, qn, sizes, d=128, scale=0.3, extra=3):
    kvh = qh // group
    kn = sizes.shape[1]
    t = int(sizes.sum(axis=1).max()) + extra
    qc = (rng.standard_normal((qh, qn, d)) * scale).astype(np.float32)
    k = rng.standard_normal((kvh, t, d)).astype(np.float32)
    v = rng.standard_normal((kvh, t, d)).astype(np.float32)
    kc = (rng.standard_normal((kvh, kn, d)) * 0.5).astype(np.float32)
    vc = (rng.standard_normal((kvh, kn, d)) * 0.5).astype(np.float32)
    return qc, k, v, kc, vc


def _brute_value_error(qc, k, v, kc, vc, sizes, group, var=None, cap=0.0):
    """exp(score) = (1/n) sum_t || e^{l_c} vc - e^{l_t} v_t ||^2 by direct vector norms: no
    expansion into |vc|^2, |v|^2, v.vc and no max shift (small logits keep e^l finite)."""
    qh, qn, d = qc.shape
    kn = sizes.shape[1]
    sc = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    out = np.full((qh, qn, kn), -np.inf)
    for h in range(qh):
        kh = h // group
        off = 0
        for c in range(kn):
            n = int(sizes[kh, c])
            if n == 0:
                continue
            for i in range(qn):
                q = qc[h, i].astype(np.float64)
                lc = float(q @ kc[kh, c]) * sc
                if cap > 0.0:
                    lc += 0.5 * min(float((q * q) @ var[kh, c]) / d, cap)
                qt = (q.astype(np.float32).view(np.uint32).astype(np.uint64) + 0x1000) & 0xFFFFE000
                qt = qt.astype(np.uint32).view(np.float32).astype(np.float64)
                tot = 0.0
                for t in range(off, off + n):
                    lt = float(qt @ k[kh, t].astype(np.float64)) * sc
                    diff = math.exp(lc) * vc[kh, c].astype(np.float64) - math.exp(lt) * v[kh, t].astype(np.float64)
                    tot += float(diff @ diff)
                out[h, i, c] = math.log(tot / n)
            off += n
    return out


@pytest.mark.parametrize("group", [1, 2])
def test_svg_ear_value_error_closed_form(oracle, group):
    rng = np.random.default_rng(7 + group)
    sizes = np.array([[3, 0, 5, 1], [2, 4, 0, 6]], np.int32)[: 2 // group]
    qc, k, v, kc, vc = _svg_case(rng, 2, group, 3, sizes)
    got = oracle.svg_ear_value_error_scores(qc, k, v, kc, vc, sizes, group).astype(np.float64)
    ref = _brute_value_error(qc, k, v, kc, vc, sizes, group)
    assert (np.isinf(got) == np.isinf(ref)).all()
    fin = np.isfinite(ref)
    assert np.abs(got[fin] - ref[fin]).max() < 1e-5


def test_svg_ear_jensen_term(oracle):
    rng = np.random.default_rng(11)
    sizes = np.array([[4, 2, 3]], np.int32)
    qc, k, v, kc, vc = _svg_case(rng, 1, 1, 4, sizes)
    var = rng.uniform(0.0, 2.0, kc.shape).astype(np.float32)
    base = oracle.svg_ear_value_error_scores(qc, k, v, kc, vc, sizes, 1)
    zero = oracle.svg_ear_value_error_scores(qc, k, v, kc, vc, sizes, 1, np.zeros_like(var), 0.5)
    assert np.array_equal(base, zero)
    for cap in (0.01, 10.0):  # the cap binding and not binding
        got = oracle.svg_ear_value_error_scores(qc, k, v, kc, vc, sizes, 1, var, cap).astype(np.float64)
        ref = _brute_value_error(qc, k, v, kc, vc, sizes, 1, var, cap)
        assert np.abs(got - ref).max() < 1e-5


def test_attention_mass_is_cluster_logsumexp(oracle):
    from scipy.special import logsumexp

    rng = np.random.default_rng(3)
    sizes = np.array([[5, 0, 9, 1, 30]], np.int32)
    qc, k, _, _, _ = _svg_case(rng, 2, 2, 6, sizes, scale=2.0)
    got = oracle.attention_mass_scores(qc, k, sizes, 2).astype(np.float64)
    sc = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    qt = oracle.tf32_rna(qc).astype(np.float64)
    off = np.concatenate(([0], np.cumsum(sizes[0])))
    for h in range(2):
        for c in range(5):
            if sizes[0, c] == 0:
                assert np.isinf(got[h, :, c]).all() and (got[h, :, c] < 0).all()
                continue
            lt = (qt[h] @ k[0, off[c]:off[c + 1]].astype(np.float64).T) * sc
            assert np.abs(got[h, :, c] - logsumexp(lt, axis=1)).max() < 1e-5


def test_role_projection_rms_closed_form(oracle):
    rng = np.random.default_rng(5)
    x = oracle.to_bf16(rng.standard_normal((2, 9, 64)).astype(np.float32))
    f = rng.standard_normal((2, 64, 48)).astype(np.float32)
    x[1, 3] = 0.0  # a zero row: p = 0, the 1e-12 floor keeps it at 0
    got = oracle.role_projection_rms(x, f).astype(np.float64)
    ft = oracle.tf32_rna(f).astype(np.float64)
    for b in range(2):
        for n in range(9):
            p = np.array([sum(float(x[b, n, d]) * ft[b, d, r] for d in range(64)) for r in range(48)])
            nrm = np.linalg.norm(p)
            want = p * math.sqrt(48) / nrm if nrm > 0 else np.zeros(48)
            assert np.abs(got[b, n] - want).max() < 1e-5
    # rows are unit RMS (except the zero row), and the projection uses the TF32 factor
    rms = np.sqrt((got ** 2).mean(axis=2))
    assert np.abs(np.delete(rms.reshape(-1), 1 * 9 + 3) - 1.0).max() < 1e-6
    assert not np.allclose(oracle.role_projection_rms(x, f), oracle.role_projection_rms(x, f + 2 ** -14 * f), atol=0)


def test_role_k_projection_head_scale(oracle):
    rng = np.random.default_rng(8)
    k = oracle.to_bf16(rng.standard_normal((3, 40, 64)).astype(np.float32))
    f = rng.standard_normal((3, 64, 32)).astype(np.float32)
    k[2] = 0.0  # an all-zero head: scale clamps at 1e-8 and the key stays 0
    key, scale = oracle.role_k_projection_normalize(k, f)
    ft = oracle.tf32_rna(f).astype(np.float64)
    for b in range(2):
        p = k[b].astype(np.float64) @ ft[b]
        s = np.linalg.norm(p) / math.sqrt(p.size)  # Frobenius norm: another route to the RMS
        assert abs(scale[b, 0, 0] - s) <= 1e-6 * s
        assert np.abs(key[b] - p / s).max() < 1e-5
    assert scale[2, 0, 0] == np.float32(1e-8) and not key[2].any()
    # scaling K by c scales the key by 1 (the head RMS normalises it away) and the scale by c
    key2, scale2 = oracle.role_k_projection_normalize(k * 4.0, f)
    assert np.abs(key2[:2] - key[:2]).max() < 1e-6 and np.abs(scale2[:2] / scale[:2] - 4.0).max() < 1e-6


# --------------------------------------------------------------------------- top-p key budgets

def test_svg_top_p_key_budgets_brute_force_walk(oracle):
    """n8_v6.py:181-230 evaluated by a per-row float64 walk written out in Python: the
    logits, max shift, weighted exponentials and normalisation by loops, a sort with
    (probability desc, index asc) keys, then the cumulative walk that keeps rank 0 and
    every rank whose preceding mass is <= p, summing the kept sizes.  Rows whose walk
    passes within 1e-6 of p are skipped (fp32 and float64 may decide them differently)."""
    rng = np.random.default_rng(31)
    bh, qn, kn, d = 2, 6, 23, 16
    qc = (0.7 * rng.standard_normal((bh, qn, d))).astype(np.float32)
    kc = (0.7 * rng.standard_normal((bh, kn, d))).astype(np.float32)
    ks = rng.integers(0, 50, (bh, kn)).astype(np.int32)
    ks[:, 3] = 0  # an empty cluster
    checked = 0
    for p in (0.3, 0.5, 0.7, 0.85, 1.0):
        got = oracle.svg_top_p_key_budgets(qc, kc, ks, p)
        assert got.dtype == np.int64 and got.shape == (bh, qn)
        for h in range(bh):
            for i in range(qn):
                logits = [sum(float(qc[h, i, t]) * float(kc[h, j, t]) for t in range(d)) / math.sqrt(d)
                          for j in range(kn)]
                mx = max(logits)
                we = [math.exp(x - mx) * float(ks[h, j]) for j, x in enumerate(logits)]
                tot = max(sum(we), 1e-12)
                order = sorted(range(kn), key=lambda j: (-we[j] / tot, j))
                budget, cum, near = 0, 0.0, False
                for r, j in enumerate(order):
                    if r > 0 and cum > p:
                        break
                    budget += int(ks[h, j])
                    cum += we[j] / tot
                    near |= abs(cum - p) < 1e-6
                if not near:
                    assert got[h, i] == budget, (p, h, i)
                    checked += 1
    assert checked >= 40
    # p = 1 keeps every cluster until the mass is exhausted: at least the largest size
    assert (oracle.svg_top_p_key_budgets(qc, kc, ks, 1.0) >= ks.max(1)[:, None]).all()


# --------------------------------------------------------------------------- multi-round probes

def test_rounds_probe_sequence_hand_derived(oracle):
    """select_role_equal_probes (residual_repair.py:36-115) with more probes than groups,
    worked by hand.  Eight tokens; groups by size: 0 = {0, 2, 4, 6, 7}, 1 = {1, 5},
    2 = {3}.  Group 0's centre is (0, 0): distances t0 0, t6 0.25, t4 1, t7 6.25, t2 9;
    group 1's centre is (10, 2.5): t1 = t5 = 2.25 (a tie: the lower id first); group 2: t3 0.
      round 1: nearest of each group in size order                      -> 0, 1, 3
      round 2: group 2 is exhausted, so its best distance is inf and every member
               (inf == inf) is a candidate: its lowest id, 3, is offered again -> 6, 5, 3
      round 3: two rows left: group 0's next, then group 1 (now exhausted)
               re-offers its lowest id 1                                       -> 4, 1
    Weights: sizes (5, 2, 1) / sampled (3, 3, 2) = (5/3, 2/3, 1/2) per group, whose mean
    over the eight rows is exactly 1."""
    f = np.zeros((1, 8, 2), np.float32)
    for t, xy in {0: (0.0, 0.0), 2: (3.0, 0.0), 4: (-1.0, 0.0), 6: (0.5, 0.0), 7: (-2.5, 0.0),
                  1: (10.0, 1.0), 5: (10.0, 4.0), 3: (-7.0, -7.0)}.items():
        f[0, t] = xy
    labels = np.array([[0, 1, 0, 2, 0, 1, 0, 0]], np.int32)
    rows, w = oracle.select_role_equal_probes(f, labels, 3, 8)
    assert rows[0].tolist() == [0, 1, 3, 6, 5, 3, 4, 1]
    per_group = {0: 5.0 / 3.0, 1: 2.0 / 3.0, 2: 0.5}
    want = np.array([per_group[int(labels[0, r])] for r in rows[0]])
    assert np.allclose(w[0], want, rtol=1e-6)
    # fewer rows than groups stops inside round 1; the count is capped at the tokens
    assert oracle.select_role_equal_probes(f, labels, 3, 2)[0][0].tolist() == [0, 1]
    assert oracle.select_role_equal_probes(f, labels, 3, 20)[0].shape == (1, 8)


# --------------------------------------------------------------------------- N8 role metrics and factors

def test_role_metric_against_numpy_cov(oracle):
    """Centred metric = np.cov(bias=True) of the used rows; uncentred = centred + mean mean^T
    (two routes to the same matrix); the size mask drops rows from the mean and the count."""
    rng = np.random.default_rng(51)
    x = (rng.standard_normal((2, 300, 8)) + 0.5).astype(np.float32)
    rows = np.array([0, 7, 19, 150, 151, 299])
    cen = oracle.role_metric(x, rows=rows, center=True)
    unc = oracle.role_metric(x, rows=rows, center=False)
    for h in range(2):
        xs = x[h, rows].astype(np.float64)
        assert np.allclose(cen[h], np.cov(xs.T, bias=True), rtol=1e-12, atol=1e-12)
        mu = xs.mean(0)
        assert np.allclose(unc[h], cen[h] + np.outer(mu, mu), rtol=1e-10, atol=1e-12)
    sizes = rng.integers(-1, 3, (2, 300))
    q = oracle.role_metric(x, sizes=sizes, center=True, post_scale=1.0 / 8)
    for h in range(2):
        xs = x[h, sizes[h] > 0].astype(np.float64)
        assert np.allclose(q[h], np.cov(xs.T, bias=True) / 8, rtol=1e-12, atol=1e-12)


def _spectrum_matrix(rng, bh, d, eig):
    qm = np.linalg.qr(rng.standard_normal((bh, d, d)))[0]
    return np.einsum("bij,j,bkj->bik", qm, eig, qm), qm


def test_metric_factor_constructed_spectrum(oracle):
    """M = Q diag(lambda) Q^T with known lambda: F F^T = sum over the top r of
    lambda_i / mean(top r, clamped) q_i q_i^T; a negative eigenvalue inside the top r gives a
    zero column; an asymmetric perturbation is removed by the symmetrisation."""
    rng = np.random.default_rng(52)
    d, r = 12, 5
    eig = np.array([-3.0, -1, 0.1, 0.2, 0.3, 0.5, 0.8, 1.3, 2.1, 3.4, 5.5, 8.9])
    m, qm = _spectrum_matrix(rng, 2, d, eig)
    skew = rng.standard_normal((2, d, d)) * 1e-3
    f = oracle.metric_factor(m + skew - np.swapaxes(skew, 1, 2), r)
    top = eig[-r:]
    want = np.einsum("bij,j,bkj->bik", qm[:, :, -r:], top / top.mean(), qm[:, :, -r:])
    assert np.allclose(np.einsum("bir,bjr->bij", f, f), want, atol=1e-9)
    neg = np.array([-5.0, -4, -3, -2, -1, 0.5, 0.7])
    m2, _ = _spectrum_matrix(rng, 1, 7, neg)
    f2 = oracle.metric_factor(m2, 3)  # top 3: -1, 0.5, 0.7 -> the -1 column is zero
    assert np.allclose(f2[0, :, 0], 0.0) and np.abs(f2[0, :, 1:]).max() > 0.1


def test_warm_subspace_factor_fixed_point(oracle):
    """Started from the exact top-r eigenvectors, subspace iteration stays on that subspace:
    F F^T = P M P / mean(diag of the Rayleigh matrix), up to the 1e-4 Rayleigh ridge; the
    Cholesky-QR basis is orthonormal; every finish gives the same subspace; a NaN metric
    marks the head recovered."""
    rng = np.random.default_rng(53)
    d, r = 16, 6
    eig = np.linspace(0.1, 1.0, d) ** 3
    eig[-r:] = [2.0, 2.5, 3.0, 4.0, 5.0, 7.0]
    m, qm = _spectrum_matrix(rng, 2, d, eig)
    prev = qm[:, :, -r:] * rng.uniform(0.5, 2.0, (2, 1, r))  # columns with arbitrary scales
    f, b, rec = oracle.warm_subspace_metric_factor(m, prev, r)
    assert not rec.any()
    proj = np.einsum("bir,bjr->bij", qm[:, :, -r:], qm[:, :, -r:])
    pmp = proj @ m @ proj
    norm = eig[-r:].mean()
    assert np.allclose(np.einsum("bir,bjr->bij", f, f), pmp / norm, atol=2e-3 * np.abs(pmp / norm).max())
    assert np.allclose(np.einsum("bir,bis->brs", b, b), np.eye(r), atol=1e-4)
    for ortho, ritz in [("each_cholesky_qr", "diagonal"), ("cholesky_qr", "previous_scale")]:
        f2, b2, _ = oracle.warm_subspace_metric_factor(m, prev, r, orthogonalization=ortho, ritz_mode=ritz)
        assert np.allclose(np.einsum("bir,bjr->bij", b2, b2), proj, atol=1e-3)
    bad = m.copy()
    bad[1, 0, 0] = np.nan
    _, _, rec = oracle.warm_subspace_metric_factor(bad, prev, r)
    assert rec.tolist() == [False, True]


def test_householder_qr_is_the_lapack_convention(oracle):
    """The reference's torch.linalg.qr is LAPACK geqrf + orgqr: R's diagonal is
    -sign(pivot) |column|, and a column already zero below its pivot takes tau = 0 (Q's
    column is e_k).  Hand-worked: [[3], [4]] -> Q = [[-0.6], [-0.8]]; [[2, 1], [0, 3], [0, 4]]
    -> Q = [[1, 0], [0, -0.6], [0, -0.8]] (H_0 = I, then v = [1, 1/2], tau = 1.6)."""
    assert np.allclose(oracle.householder_qr(np.array([[3.0], [4.0]])), [[-0.6], [-0.8]], atol=1e-15)
    got = oracle.householder_qr(np.array([[2.0, 1.0], [0.0, 3.0], [0.0, 4.0]]))
    assert np.allclose(got, [[1.0, 0.0], [0.0, -0.6], [0.0, -0.8]], atol=1e-15)
    rng = np.random.default_rng(55)
    a = rng.standard_normal((9, 4))
    q = oracle.householder_qr(a)
    r = q.T @ a
    assert np.allclose(q.T @ q, np.eye(4), atol=1e-12) and np.allclose(np.tril(r, -1), 0.0, atol=1e-12)
    assert np.sign(r[0, 0]) == -np.sign(a[0, 0])


def test_warm_subspace_factor_householder_and_full_ritz(oracle):
    """each_qr / final_qr (operator_kmeans.py:366-371, :405-419) and the full Rayleigh-Ritz
    finish (:460-466).  Started on the exact top-r eigenvectors: the full finish gives
    F F^T = P M P / mean(top eigenvalues) exactly (no ridge), its columns are orthogonal with
    squared norms the top eigenvalues / their mean in ascending order, and a negative
    eigenvalue inside the subspace is clamped to a zero column (and out of the mean).  Each
    basis is orthonormal; one each_qr step is the QR of M Q(prev) (B^T M Q(prev) upper
    triangular); final_qr's basis spans M^p prev; from a random start many steps converge
    to the top subspace."""
    rng = np.random.default_rng(56)
    d, r = 16, 6
    eig = np.linspace(0.1, 1.0, d) ** 3
    eig[-r:] = [2.0, 2.5, 3.0, 4.0, 5.0, 7.0]
    m, qm = _spectrum_matrix(rng, 2, d, eig)
    top = qm[:, :, -r:]
    proj = np.einsum("bir,bjr->bij", top, top)
    pmp = proj @ m @ proj
    prev = top * rng.uniform(0.5, 2.0, (2, 1, r))
    for ortho in ("each_qr", "final_qr", "each_cholesky_qr2"):
        f, b, rec = oracle.warm_subspace_metric_factor(m, prev, r, orthogonalization=ortho, ritz_mode="full")
        assert not rec.any()
        assert np.allclose(np.einsum("bir,bjr->bij", f, f), pmp / eig[-r:].mean(), atol=1e-9)
        assert np.allclose(np.einsum("bir,bis->brs", b, b), np.eye(r), atol=1e-9)
        assert np.allclose(np.einsum("bir,bis->brs", f, f), np.stack([np.diag(eig[-r:] / eig[-r:].mean())] * 2),
                           atol=1e-9)
    # one each_qr step from a random start is the QR of M Q(prev); final_qr spans M^p prev
    prev_r = rng.standard_normal((2, d, r))
    _, b1, _ = oracle.warm_subspace_metric_factor(m, prev_r, r, power_iters=1, orthogonalization="each_qr",
                                                  ritz_mode="previous_scale")
    for h in range(2):
        q0, _ = np.linalg.qr(prev_r[h])
        tri = b1[h].T @ (m[h] @ q0)
        assert np.allclose(np.tril(tri, -1), 0.0, atol=1e-10) and np.allclose(b1[h].T @ b1[h], np.eye(r), atol=1e-12)
    _, b3, _ = oracle.warm_subspace_metric_factor(m, prev_r, r, power_iters=3, orthogonalization="final_qr",
                                                  ritz_mode="previous_scale")
    for h in range(2):
        target = np.linalg.matrix_power(m[h], 3) @ prev_r[h]
        resid = target - b3[h] @ (b3[h].T @ target)
        assert np.linalg.norm(resid) <= 1e-10 * np.linalg.norm(target)
    fc, _, _ = oracle.warm_subspace_metric_factor(m, prev_r, r, power_iters=60, orthogonalization="each_qr",
                                                  ritz_mode="full")
    assert np.allclose(np.einsum("bir,bjr->bij", fc, fc), pmp / eig[-r:].mean(), atol=1e-8)
    # a negative eigenvalue inside the tracked subspace: that column is zero, the mean skips it
    eig2 = eig.copy()
    eig2[-r] = -1.5
    m2, qm2 = _spectrum_matrix(rng, 1, d, eig2)
    f2, _, _ = oracle.warm_subspace_metric_factor(m2, qm2[:, :, -r:], r, orthogonalization="each_qr",
                                                  ritz_mode="full")
    norms2 = (f2[0] ** 2).sum(0)
    kept = np.sort(eig2[-r:])[1:]
    assert np.allclose(norms2, np.concatenate(([0.0], kept / (kept.sum() / r))), atol=1e-9)


def test_svg_ear_compensation_closed_forms(oracle):
    """svg_ear.py:289-369.  Every cluster selected: the sparse output comes back exactly, in
    both reformulations.  No cluster selected and one valid cluster (count 4, tf32-exact
    values): out = (s e^lse + 4 e^(q.kc / sqrt D) vc) / (e^lse + 4 e^(q.kc / sqrt D)), worked
    by hand.  An empty cluster (count 0) adds nothing.  n3_residual equals skipped on random
    masks (the same sum in exact arithmetic, up to the TF32 rounding of the weights).  A row with lse = -inf whose first block has no
    cluster to add stays NaN, as the reference's exp(-inf - -inf) makes it."""
    d = 4
    q = np.array([[[2.0, 0.0, 0.0, 0.0]]], np.float32)
    sparse = np.array([[[1.0, 2.0, 3.0, 4.0]]], np.float32)
    lse = np.array([[0.5]], np.float32)
    kc = np.array([[[1.0, 0.0, 0.0, 0.0], [3.0, 1.0, 0.0, 0.0]]], np.float32)
    vc = np.array([[[8.0, 0.0, -8.0, 0.0], [5.0, 5.0, 5.0, 5.0]]], np.float32)
    counts = np.array([[4.0, 0.0]], np.float32)
    labels = np.zeros((1, 1), np.int64)
    none = np.zeros((1, 2, 3), bool)
    allsel = np.ones((1, 2, 3), bool)
    for ref in ("skipped", "n3_residual"):
        same = oracle.svg_ear_compensation(q, sparse, lse, labels, allsel, kc, counts, vc, ref)
        assert np.array_equal(same, sparse)
        got = oracle.svg_ear_compensation(q, sparse, lse, labels, none, kc, counts, vc, ref)
        l0 = 2.0 / 2.0 + np.log(4.0)  # q.kc / sqrt(4) + log(count)
        want = (sparse[0, 0] * np.exp(0.5) + np.exp(l0) * vc[0, 0]) / (np.exp(0.5) + np.exp(l0))
        assert np.allclose(got[0, 0], want, rtol=1e-6)
    rng = np.random.default_rng(57)
    bh, t, kn, d = 2, 20, 70, 16
    qr = rng.standard_normal((bh, t, d)).astype(np.float32)
    sp = rng.standard_normal((bh, t, d)).astype(np.float32)
    ls = rng.standard_normal((bh, t)).astype(np.float32)
    lab = rng.integers(0, 5, (bh, t))
    dm = rng.random((bh, 6, kn + 1)) < 0.4
    kcr = rng.standard_normal((bh, kn, d)).astype(np.float32)
    vcr = rng.standard_normal((bh, kn, d)).astype(np.float32)
    cnt = rng.integers(0, 9, (bh, kn)).astype(np.float32)
    a = oracle.svg_ear_compensation(qr, sp, ls, lab, dm, kcr, cnt, vcr, "skipped")
    b = oracle.svg_ear_compensation(qr, sp, ls, lab, dm, kcr, cnt, vcr, "n3_residual")
    # equal up to the TF32 rounding of the weights (their scale follows each mode's running max)
    assert np.abs(a - b).max() <= 2e-3 * np.abs(a).max()
    ls2 = ls.copy()
    ls2[0, 0] = -np.inf
    dm2 = dm.copy()
    dm2[0, lab[0, 0] + 1, 1:33] = True  # nothing to add in the first block
    nan = oracle.svg_ear_compensation(qr, sp, ls2, lab, dm2, kcr, cnt, vcr, "skipped")
    assert np.isnan(nan[0, 0]).all() and np.isfinite(nan[0, 1:]).all()


def test_project_rows_loop(oracle):
    rng = np.random.default_rng(54)
    x = rng.standard_normal((1, 5, 8)).astype(np.float32)
    f = rng.standard_normal((1, 8, 3)).astype(np.float32)
    got = oracle.project_rows(x, f, div=np.array([2.0]), tf32=True)
    for i in range(5):
        for c in range(3):
            want = sum(float(a) * float(b) for a, b in zip(oracle.tf32_rna(x[0, i]), oracle.tf32_rna(f[0, :, c])))
            assert abs(got[0, i, c] - want / 2.0) < 1e-12
    rms = oracle.project_rows(x, f, row_rms=True)
    assert np.allclose(np.sqrt((rms ** 2).mean(-1)), 1.0)


# ---------------------------------------------------------------- QKV norm + RoPE fusions

def test_wan_qkv_oracle_pins(oracle):
    """Wan's RoPE as complex multiplication of adjacent channel pairs (an independent
    numpy-complex formulation), the RMSNorm's unit RMS and scale invariance, the identity
    at angle 0 and the exact quarter turn, and the BHLD layout of V."""
    rng = np.random.default_rng(71)
    b, l, h, d = 2, 7, 3, 8
    c = h * d
    q = rng.standard_normal((b, l, c)) * 3.0
    k = rng.standard_normal((b, l, c))
    v = rng.standard_normal((b, l, c))
    w = rng.uniform(0.5, 1.5, c)
    ang = rng.uniform(-3, 3, (l, d // 2))
    qo, ko, vo = oracle.wan_qkv_norm_rope_layout(q, k, v, w, w, np.cos(ang), np.sin(ang), h, 1e-6, dtype="fp64")
    rms = np.sqrt((q * q).mean(-1, keepdims=True) + 1e-6)
    z = ((q / rms * w).reshape(b, l, h, d // 2, 2) @ np.array([1.0, 1j])) * np.exp(1j * ang)[None, :, None, :]
    want = np.stack((z.real, z.imag), -1).reshape(b, l, h, d).transpose(0, 2, 1, 3)
    assert np.allclose(qo, want, rtol=1e-12, atol=1e-12)
    assert np.array_equal(vo, v.reshape(b, l, h, d).transpose(0, 2, 1, 3))
    ones = np.ones(c)
    q1, _, _ = oracle.wan_qkv_norm_rope_layout(q, k, v, ones, ones, np.ones((l, d // 2)), np.zeros((l, d // 2)),
                                               h, 0.0, dtype="fp64")
    assert np.allclose((q1 ** 2).transpose(0, 2, 1, 3).reshape(b, l, c).mean(-1), 1.0)  # unit RMS per token
    q2, _, _ = oracle.wan_qkv_norm_rope_layout(5.0 * q, k, v, ones, ones, np.ones((l, d // 2)),
                                               np.zeros((l, d // 2)), h, 0.0, dtype="fp64")
    assert np.allclose(q1, q2)
    # quarter turn: (x0, x1) -> (-x1, x0), exact in bf16
    qb, _, _ = oracle.wan_qkv_norm_rope_layout(q, k, v, w, w, np.zeros((l, d // 2)), np.ones((l, d // 2)), h, 1e-6)
    qn, _, _ = oracle.wan_qkv_norm_rope_layout(q, k, v, w, w, np.ones((l, d // 2)), np.zeros((l, d // 2)), h, 1e-6)
    assert np.array_equal(qb[..., 0::2], -qn[..., 1::2]) and np.array_equal(qb[..., 1::2], qn[..., 0::2])


def test_cosmos_qkv_oracle_pins(oracle):
    """Cosmos's rotate-half RoPE equals complex multiplication of the pairs (d, d + D/2) when
    the angle table repeats its halves (Transformer Engine's layout); a rotation keeps each
    pair's norm and the inverse angle undoes it; per-head unit RMS; the quarter turn."""
    rng = np.random.default_rng(72)
    b, s_len, h, d = 2, 5, 3, 16
    half = d // 2
    q = rng.standard_normal((b, s_len, h * d)) * 2.0
    k = rng.standard_normal((b, s_len, h * d))
    v = rng.standard_normal((b, s_len, h * d))
    w = rng.uniform(0.5, 1.5, d)
    freqs = rng.uniform(-3, 3, (s_len, half))
    ang = np.concatenate((freqs, freqs), -1).reshape(s_len, 1, 1, d)
    qo, _, vo = oracle.cosmos25_qkv_norm_rope_bshd(q, k, v, w, w, ang, h, 1e-6, dtype="fp64")
    x = q.reshape(b, s_len, h, d)
    r = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w
    z = (r[..., :half] + 1j * r[..., half:]) * np.exp(1j * freqs)[None, :, None, :]
    assert np.allclose(qo, np.concatenate((z.real, z.imag), -1), rtol=1e-12, atol=1e-12)
    assert np.array_equal(vo, v.reshape(b, s_len, h, d))
    assert np.allclose(np.hypot(qo[..., :half], qo[..., half:]), np.hypot(r[..., :half], r[..., half:]))
    back, _, _ = oracle.cosmos25_qkv_norm_rope_bshd(qo.reshape(b, s_len, h * d), k, v, np.ones(d), np.ones(d),
                                                    -ang, h, 0.0, dtype="fp64")
    rn = r / np.sqrt((r * r).mean(-1, keepdims=True))
    assert np.allclose(back, rn)
    ones = np.ones(d)
    q1, _, _ = oracle.cosmos25_qkv_norm_rope_bshd(q, k, v, ones, ones, np.zeros((s_len, 1, 1, d)), h, 0.0,
                                                  dtype="fp64")
    assert np.allclose((q1 ** 2).mean(-1), 1.0)
    qt, _, _ = oracle.cosmos25_qkv_norm_rope_bshd(q, k, v, w, w, np.full((s_len, 1, 1, d), np.pi / 2), h, 1e-6)
    qz, _, _ = oracle.cosmos25_qkv_norm_rope_bshd(q, k, v, w, w, np.zeros((s_len, 1, 1, d)), h, 1e-6)
    # cos(pi/2) is 6e-17, below half an ulp of any of these values
    assert np.array_equal(qt[..., :half], -qz[..., half:]) and np.array_equal(qt[..., half:], qz[..., :half])


def test_matmul_precision_operands_and_joint_features(oracle):
    """The fp32 matmul precisions as operand roundings: "medium" rounds to bf16 as torch's
    bfloat16 conversion does, "high" to TF32, "highest" not at all; the joint K/V features put
    the K features first and give the V half an RMS of exactly v_weight over the head."""
    import torch

    rng = np.random.default_rng(47)
    x = (rng.standard_normal((3, 40)) * 10.0 ** rng.uniform(-3, 3, (3, 40))).astype(np.float32)
    assert (oracle.matmul_precision_operand(x, "medium") == torch.from_numpy(x).to(torch.bfloat16).float().numpy()).all()
    assert (oracle.matmul_precision_operand(x, "highest") == x).all()
    assert (oracle.matmul_precision_operand(x, "high") == oracle.tf32_rna(x)).all()
    k = oracle.to_bf16(rng.standard_normal((2, 300, 32)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((2, 300, 32)).astype(np.float32))
    kf = rng.standard_normal((2, 32, 12)).astype(np.float32)
    vf = rng.standard_normal((2, 32, 4)).astype(np.float32)
    feats, ks, vs = oracle.role_kv_projection_normalize(k, v, kf, vf, 0.25, "highest")
    assert feats.shape == (2, 300, 16)
    assert np.allclose(feats[:, :, :12], oracle.role_k_projection_normalize(k, kf, "highest")[0])
    rms_v = np.sqrt((feats[:, :, 12:].astype(np.float64) ** 2).mean(axis=(1, 2)))
    assert np.allclose(rms_v, 0.25, rtol=1e-6)
    # a direct loop for one entry: (w * sum_d k v_f) / vs
    p = sum(float(v[1, 7, j]) * float(vf[1, j, 2]) for j in range(32))
    assert abs(feats[1, 7, 14] - 0.25 * p / float(vs[1, 0, 0])) <= 1e-6 * max(abs(feats[1, 7, 14]), 1e-6)
