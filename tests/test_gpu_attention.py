"""GPU parity: block-sparse attention over cluster-pair blocks and the dense
probe attention.  Tolerance (bf16 in/out, fp32 softmax): max-abs <= 2e-2 and
cosine >= 0.999 against the float64 closed form; all-dropped rows exactly 0."""

import math

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

ATOL = 2e-2
COS = 0.999


def _cos(a, b):
    a = a.reshape(-1).astype(np.float64)
    b = b.reshape(-1).astype(np.float64)
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-30))


def _sizes(rng, n, total, empty_every=0):
    w = rng.random(n) + 0.05
    if empty_every and n > empty_every:
        w[::empty_every] = 0.0
    s = np.floor(w / w.sum() * total).astype(np.int64)
    s[np.argmax(w)] += total - s.sum()
    return s


def _problem(oracle, rng, B, Hq, Hkv, S, D, qn, kn, density=0.3, empty_row=True, scale=1.0):
    q = oracle.to_bf16((scale * rng.standard_normal((B, Hq, S, D))).astype(np.float32))
    k = oracle.to_bf16((scale * rng.standard_normal((B, Hkv, S, D))).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    qs = np.stack([[_sizes(rng, qn, S, 5) for _ in range(Hkv)] for _ in range(B)])
    ks = np.stack([[_sizes(rng, kn, S, 7) for _ in range(Hkv)] for _ in range(B)])
    m = rng.random((B, Hkv, qn, kn)) < density
    m[..., 0, 0] = True
    if empty_row and qn > 1:
        m[..., 1, :] = False
    return q, k, v, m, qs, ks


def _reference(oracle, q, k, v, m, qs, ks):
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    rep = lambda a: np.repeat(a, g, axis=1)
    return oracle.block_sparse_attention_dense(q, rep(k), rep(v), rep(m), rep(qs), rep(ks), return_lse=True)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,qn,kn", [
    (1, 2, 2, 700, 128, 6, 11),
    (1, 3, 3, 1000, 64, 9, 40),
    (2, 2, 2, 513, 128, 3, 17),     # q-clusters of > 128 rows: several tiles per cluster
    (1, 4, 2, 600, 128, 5, 9),      # GQA group 2
    (1, 1, 1, 64, 128, 1, 1),
    (1, 2, 2, 3000, 128, 6, 1024),  # kn > 768: segment lists read from the plan, not LDS
    (1, 1, 1, 2000, 64, 4, 900),    # the same for the D = 64 kernel
])
def test_block_sparse_matches_closed_form(dev, oracle, B, Hq, Hkv, S, D, qn, kn):
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    rng = np.random.default_rng(S + D + qn)
    q, k, v, m, qs, ks = _problem(oracle, rng, B, Hq, Hkv, S, D, qn, kn)
    out, lse = dynamic_block_sparse_fwd_flashinfer(
        to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16), to_dev(v, dev, torch.bfloat16),
        torch.from_numpy(m), torch.from_numpy(qs).int(), torch.from_numpy(ks).int(), is_cpu=True,
        num_kv_heads=Hkv if Hkv != Hq else None, return_lse=True)
    ref, ref_lse = _reference(oracle, q, k, v, m, qs, ks)
    got = out.float().cpu().numpy()
    assert np.abs(got - ref).max() <= ATOL
    assert _cos(got, ref) >= COS
    g = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.allclose(g[fin], ref_lse[fin], atol=1e-3, rtol=1e-4)
    assert np.isneginf(g[~fin]).all()
    # rows of q-cluster 1 (all blocks dropped) are exactly zero
    if qn > 1:
        for b in range(B):
            for h in range(Hq):
                r0 = int(qs[b, h // (Hq // Hkv), :1].sum())
                r1 = r0 + int(qs[b, h // (Hq // Hkv), 1])
                assert (got[b, h, r0:r1] == 0).all()


@pytest.mark.parametrize("D,f16,Hq,Hkv", [(16, False, 2, 2), (32, False, 4, 2), (16, True, 2, 2), (32, True, 2, 2),
                                         (64, True, 4, 2), (128, True, 2, 2)])
def test_block_sparse_head_dims_and_fp16(dev, oracle, D, f16, Hq, Hkv):
    """The head dims the reference's Triton path takes besides 64 and 128 (16 and 32:
    kmeans_utils.py:1847-2161) and fp16 Q/K/V (fp16 P and output, as a float16 call of the
    reference computes), against the float64 closed form of the same rounded inputs:
    max-abs 2e-2, cosine 0.999, LSE 1e-3; all-dropped rows exactly 0."""
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    rng = np.random.default_rng(D + 7 * f16 + Hq)
    S, qn, kn = 700, 6, 11
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, Hq, Hkv, S, D, qn, kn)
    tdt = torch.float16 if f16 else torch.bfloat16
    if f16:  # fresh values rounded to fp16 (the bf16 ones would not use fp16's mantissa)
        q, k, v = (rng.standard_normal(a.shape).astype(np.float16).astype(np.float32) for a in (q, k, v))
    out, lse = dynamic_block_sparse_fwd_flashinfer(
        to_dev(q, dev, tdt), to_dev(k, dev, tdt), to_dev(v, dev, tdt), torch.from_numpy(m),
        torch.from_numpy(qs).int(), torch.from_numpy(ks).int(), is_cpu=True,
        num_kv_heads=Hkv if Hkv != Hq else None, return_lse=True)
    assert out.dtype == tdt and out.shape == (1, Hq, S, D)
    ref, ref_lse = _reference(oracle, q, k, v, m, qs, ks)
    got = out.float().cpu().numpy()
    assert np.abs(got - ref).max() <= ATOL
    assert _cos(got, ref) >= COS
    g = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.allclose(g[fin], ref_lse[fin], atol=1e-3, rtol=1e-4)
    assert np.isneginf(g[~fin]).all()
    for h in range(Hq):
        r0 = int(qs[0, h // (Hq // Hkv), :1].sum())
        r1 = r0 + int(qs[0, h // (Hq // Hkv), 1])
        assert (got[0, h, r0:r1] == 0).all()


@pytest.mark.parametrize("D,f16,out", [(16, False, torch.float32), (32, True, torch.float16),
                                       (128, True, torch.float32), (64, True, torch.bfloat16)])
def test_dense_probe_attention_head_dims_and_fp16(dev, oracle, D, f16, out):
    from sparsepr_amd.kernels.attention import dense_attention

    rng = np.random.default_rng(D + f16)
    tdt = torch.float16 if f16 else torch.bfloat16
    rnd = (lambda a: a.astype(np.float16).astype(np.float32)) if f16 else oracle.to_bf16
    q = rnd(rng.standard_normal((3, 100, D)).astype(np.float32))
    k = rnd(rng.standard_normal((3, 1500, D)).astype(np.float32))
    v = rnd(rng.standard_normal((3, 1500, D)).astype(np.float32))
    got = dense_attention(to_dev(q, dev, tdt), to_dev(k, dev, tdt), to_dev(v, dev, tdt), nsplit=3, out_dtype=out)
    assert got.dtype == out
    ref = oracle.dense_attention(q, k, v)
    g = got.float().cpu().numpy()
    assert np.abs(g - ref).max() <= 1e-2 and _cos(g, ref) >= 0.9999


def test_block_sparse_matches_reference_loop(dev, oracle):
    """Against the loop-faithful restatement of dynamic_block_sparse_fwd_torch."""
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_triton

    rng = np.random.default_rng(7)
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, 2, 2, 400, 64, 4, 8)
    loop = oracle.block_sparse_attention_loop(q, k, v, m, qs, ks)
    out = dynamic_block_sparse_fwd_triton(to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16),
                                          to_dev(v, dev, torch.bfloat16), to_dev(m, dev), to_dev(qs, dev),
                                          to_dev(ks, dev))
    got = out.float().cpu().numpy()
    assert np.abs(got - loop).max() <= ATOL and _cos(got, loop) >= COS


def test_block_sparse_full_map_equals_dense(dev, oracle):
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    rng = np.random.default_rng(8)
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, 2, 2, 333, 128, 4, 6, empty_row=False)
    m[:] = True
    out = dynamic_block_sparse_fwd_flashinfer(to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16),
                                              to_dev(v, dev, torch.bfloat16), to_dev(m, dev), to_dev(qs, dev),
                                              to_dev(ks, dev), is_cpu=False)
    ref = oracle.dense_attention(q[0], k[0], v[0])
    got = out[0].float().cpu().numpy()
    assert np.abs(got - ref).max() <= ATOL and _cos(got, ref) >= COS


def test_plan_cache_reuse(dev, oracle):
    from sparsepr_amd.kernels.attention import clear_plan_cache
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    rng = np.random.default_rng(9)
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, 2, 2, 300, 128, 3, 5)
    args = [to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16), to_dev(v, dev, torch.bfloat16)]
    o1 = dynamic_block_sparse_fwd_flashinfer(*args, to_dev(m, dev), to_dev(qs, dev), to_dev(ks, dev), is_cpu=False,
                                             plan_cache_key="layer0", plan_cache_token=1)
    o2 = dynamic_block_sparse_fwd_flashinfer(*args, to_dev(m, dev), to_dev(qs, dev), to_dev(ks, dev), is_cpu=False,
                                             plan_cache_key="layer0", plan_cache_token=1)
    assert torch.equal(o1, o2)
    with pytest.raises(ValueError):
        dynamic_block_sparse_fwd_flashinfer(*args, to_dev(m, dev), to_dev(qs, dev), to_dev(ks, dev), is_cpu=False,
                                            plan_cache_key="layer0")
    clear_plan_cache()


@pytest.mark.parametrize("M,S,D,nsplit", [(128, 5000, 128, None), (64, 4096, 64, 3), (200, 1000, 128, 1),
                                          (17, 777, 128, 5)])
def test_dense_probe_attention(dev, oracle, M, S, D, nsplit):
    from sparsepr_amd.kernels.attention import dense_attention

    rng = np.random.default_rng(M + S)
    q = oracle.to_bf16(rng.standard_normal((3, M, D)).astype(np.float32))
    k = oracle.to_bf16(rng.standard_normal((3, S, D)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((3, S, D)).astype(np.float32))
    out, lse = dense_attention(to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16),
                               to_dev(v, dev, torch.bfloat16), nsplit=nsplit, return_lse=True)
    ref = oracle.dense_attention(q, k, v)
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 5e-3 and _cos(got, ref) >= 0.9999
    s = np.einsum("bmd,bsd->bms", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(D)
    ref_lse = np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
    assert np.allclose(lse.cpu().numpy(), ref_lse, atol=2e-3)


@pytest.mark.parametrize("M,S,nsplit", [(300, 3000, 4), (300, 10, 8)])
def test_dense_probe_attention_gqa_tiles(dev, oracle, M, S, nsplit):
    """D = 128 with query heads sharing key heads (6 on 2), more rows than one 256-row
    tile, a key count that is not a multiple of the 64-key chunk, and (S = 10 over 8
    splits) key splits with no keys at all."""
    from sparsepr_amd.kernels.attention import dense_attention

    rng = np.random.default_rng(M * S)
    q = oracle.to_bf16(rng.standard_normal((6, M, 128)).astype(np.float32))
    k = oracle.to_bf16(rng.standard_normal((2, S, 128)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((2, S, 128)).astype(np.float32))
    out, lse = dense_attention(to_dev(q, dev, torch.bfloat16), to_dev(k, dev, torch.bfloat16),
                               to_dev(v, dev, torch.bfloat16), nsplit=nsplit, return_lse=True)
    kk, vv = np.repeat(k, 3, 0), np.repeat(v, 3, 0)
    ref = oracle.dense_attention(q, kk, vv)
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 5e-3 and _cos(got, ref) >= 0.9999
    s = np.einsum("bmd,bsd->bms", q.astype(np.float64), kk.astype(np.float64)) / math.sqrt(128)
    ref_lse = np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
    assert np.allclose(lse.cpu().numpy(), ref_lse, atol=2e-3)


def test_dense_probe_attention_reads_a_key_slice_in_place(dev, oracle):
    """K/V given as the first S keys of a longer packed tensor (the probes attend the video
    keys plus the prompt): read in place through the head stride, the output is the same
    bits as from packed copies, and matches the float64 closed form."""
    from sparsepr_amd.kernels.attention import dense_attention

    rng = np.random.default_rng(77)
    full = 1300
    q = oracle.to_bf16(rng.standard_normal((4, 64, 128)).astype(np.float32))
    kf = oracle.to_bf16(rng.standard_normal((4, full, 128)).astype(np.float32))
    vf = oracle.to_bf16(rng.standard_normal((4, full, 128)).astype(np.float32))
    dk, dv = to_dev(kf, dev, torch.bfloat16), to_dev(vf, dev, torch.bfloat16)
    for s_kv in (1000, 1077):
        ks, vs = dk[:, :s_kv], dv[:, :s_kv]
        assert not ks.is_contiguous()
        got = dense_attention(to_dev(q, dev, torch.bfloat16), ks, vs)
        packed = dense_attention(to_dev(q, dev, torch.bfloat16), ks.contiguous(), vs.contiguous())
        assert torch.equal(got, packed)
        ref = oracle.dense_attention(q, kf[:, :s_kv], vf[:, :s_kv])
        assert np.abs(got.cpu().numpy() - ref).max() <= 5e-3


def test_block_sparse_full_size_sampled_rows(dev, oracle):
    """HunyuanVideo shape (24 heads x 118,800 x 128): a random map over 128 x 512
    cluster pairs; 192 sampled rows checked against float64 on the CPU."""
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    H, S, D, qn, kn = 24, 118800, 128, 128, 512
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    q = torch.randn(1, H, S, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(1, H, S, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, H, S, D, device=dev, generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(4)
    qs = np.stack([_sizes(rng, qn, S, 0) for _ in range(H)])[None]
    ks = np.stack([_sizes(rng, kn, S, 50) for _ in range(H)])[None]
    m = rng.random((1, H, qn, kn)) < 0.12
    out = dynamic_block_sparse_fwd_flashinfer(q, k, v, to_dev(m, dev), to_dev(qs, dev), to_dev(ks, dev),
                                              is_cpu=False)
    qoff = np.concatenate([np.zeros((1, H, 1), np.int64), np.cumsum(qs, -1)], -1)
    koff = np.concatenate([np.zeros((1, H, 1), np.int64), np.cumsum(ks, -1)], -1)
    for _ in range(192):
        h = int(rng.integers(0, H))
        r = int(rng.integers(0, S))
        a = int(np.searchsorted(qoff[0, h], r, side="right") - 1)
        keys = np.concatenate([np.arange(koff[0, h, c], koff[0, h, c + 1]) for c in np.nonzero(m[0, h, a])[0]]
                              + [np.zeros(0, np.int64)])
        got = out[0, h, r].float().cpu().numpy()
        if keys.size == 0:
            assert (got == 0).all()
            continue
        kk = k[0, h, torch.from_numpy(keys).to(dev)].double().cpu().numpy()
        vv = v[0, h, torch.from_numpy(keys).to(dev)].double().cpu().numpy()
        s = kk @ q[0, h, r].double().cpu().numpy() / math.sqrt(D)
        e = np.exp(s - s.max())
        ref = (e / e.sum()) @ vv
        assert np.abs(got - ref).max() <= ATOL


def test_q_index_fuses_the_query_permutation(dev, oracle):
    """Reading Q and writing O through the query sort index equals permute ->
    attention -> inverse permute exactly (same rows, same arithmetic)."""
    from sparsepr_amd.kernels.attention import block_sparse_attention
    from sparsepr_amd.kernels.permute import apply_inverse_permutation_triton, permute_tensor_by_labels_triton

    rng = np.random.default_rng(21)
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, 4, 2, 900, 128, 7, 13)
    q, k, v, m, ks = q[0], k[0], v[0], m[0], ks[0]
    bh_q, s, d = q.shape
    labels = np.repeat(np.arange(7), qs[0][0])[None, :].repeat(bh_q, 0)
    for h in range(bh_q):  # tokens of each q-cluster scattered over the sequence
        labels[h] = labels[h][rng.permutation(s)]
    labels_t = to_dev(labels.astype(np.int32), dev)
    qd = to_dev(q, dev, torch.bfloat16)
    q_perm, idx = permute_tensor_by_labels_triton(qd.unsqueeze(0), labels_t.unsqueeze(0), 2)
    sizes = torch.from_numpy(np.stack([np.bincount(labels[h], minlength=7) for h in range(bh_q)]).astype(np.int32))
    args = (to_dev(k, dev, torch.bfloat16), to_dev(v, dev, torch.bfloat16), to_dev(m, dev), sizes[::2].to(dev),
            to_dev(ks, dev))
    ref_sorted, ref_lse = block_sparse_attention(q_perm[0], *args, return_lse=True)
    ref = apply_inverse_permutation_triton(ref_sorted.unsqueeze(0), idx, 2)[0]
    qi = idx.reshape(bh_q, s)
    got, lse = block_sparse_attention(qd, *args, return_lse=True, q_index=qi)
    assert torch.equal(got, ref)
    inv = torch.empty_like(qi)
    inv.scatter_(1, qi.long(), torch.arange(s, device=dev, dtype=torch.int32).expand(bh_q, -1).contiguous())
    assert torch.equal(lse, torch.gather(ref_lse, 1, inv.long()))
    # keys in token order, read through the key sort index
    bh_kv = k.shape[0]
    kperm = np.stack([rng.permutation(s) for _ in range(bh_kv)]).astype(np.int32)  # sorted position -> token
    k_tok = np.empty_like(k)
    v_tok = np.empty_like(v)
    for h in range(bh_kv):
        k_tok[h, kperm[h]] = k[h]
        v_tok[h, kperm[h]] = v[h]
    got2 = block_sparse_attention(qd, to_dev(k_tok, dev, torch.bfloat16), to_dev(v_tok, dev, torch.bfloat16),
                                  *args[2:], q_index=qi, k_index=to_dev(kperm, dev))
    assert torch.equal(got2, ref)


def test_run_rejects_a_plan_for_other_sizes(dev, oracle):
    """A plan buffer too small for the run's sizes is refused on the host (status 3); a
    plan built for another sequence length is seen by the kernels' header check, which
    writes NaN over the whole output and LSE (D = 128 and D = 64 kernels); the Python
    wrapper refuses such a plan before any launch."""
    from sparsepr_amd import _lib
    from sparsepr_amd.kernels.attention import plan_block_sparse

    rng = np.random.default_rng(11)
    q, k, v, m, qs, ks = _problem(oracle, rng, 1, 2, 2, 500, 128, 4, 8, empty_row=False)
    qd, kd, vd = (to_dev(a[0], dev, torch.bfloat16) for a in (q, k, v))
    plan = plan_block_sparse(to_dev(m[0], dev), to_dev(qs[0], dev), to_dev(ks[0], dev), 500)
    lib = _lib.load()
    stream = _lib.stream(dev)
    out = torch.full_like(qd, 7.0)
    # too small for qn=4, kn=16: refused before any launch
    st = lib.spr_block_sparse_attention_run(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), plan.data_ptr(),
                                            plan.numel(), 2, 2, 500, 128, 4, 16, 0.1, None, None, out.data_ptr(),
                                            None, stream)
    assert st == 3 and b"plan buffer" in lib.spr_last_error()
    # built for s = 500, run over the first 400 rows: the header does not match
    q4, k4, v4 = (t[:, :400].contiguous() for t in (qd, kd, vd))
    out4 = torch.full_like(q4, 7.0)
    lse4 = torch.zeros((2, 400), device=dev)
    st = lib.spr_block_sparse_attention_run(q4.data_ptr(), k4.data_ptr(), v4.data_ptr(), plan.data_ptr(),
                                            plan.numel(), 2, 2, 400, 128, 4, 8, 0.1, None, None, out4.data_ptr(),
                                            lse4.data_ptr(), stream)
    torch.cuda.synchronize()
    assert st == 0
    assert bool(torch.isnan(out4).all()) and bool(torch.isnan(lse4).all())
    q64 = q4[:, :, :64].contiguous()
    out64 = torch.full_like(q64, 7.0)
    st = lib.spr_block_sparse_attention_run(q64.data_ptr(), q64.data_ptr(), q64.data_ptr(), plan.data_ptr(),
                                            plan.numel(), 2, 2, 400, 64, 4, 8, 0.1, None, None, out64.data_ptr(),
                                            None, stream)
    torch.cuda.synchronize()
    assert st == 0 and bool(torch.isnan(out64).all())
    from sparsepr_amd.kernels.attention import block_sparse_attention

    with pytest.raises(RuntimeError, match="plan was built for"):
        block_sparse_attention(q4, k4, v4, to_dev(m[0], dev), to_dev(qs[0], dev), to_dev(ks[0], dev), plan=plan)
    # the matching run writes every row
    st = lib.spr_block_sparse_attention_run(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), plan.data_ptr(),
                                            plan.numel(), 2, 2, 500, 128, 4, 8, 0.1, None, None, out.data_ptr(),
                                            None, stream)
    torch.cuda.synchronize()
    assert st == 0 and not bool((out == 7.0).all(dim=-1).any())


@pytest.mark.parametrize("kn", [40, 900])  # 900: the segment list stays in global memory
def test_plan_from_schedule_matches_map(dev, oracle, kn):
    """The selector schedule as the attention's work list: the plan from compacted ids and
    counts gives bit-identical output to the plan from the map; a schedule with unsorted,
    duplicate and out-of-range entries acts as the map of the entries above every earlier
    entry of their row (checked against the float64 closed form too)."""
    from sparsepr_amd.kernels.attention import (block_sparse_attention, plan_block_sparse,
                                                plan_block_sparse_from_schedule)
    from sparsepr_amd.kernels.n8_extension import compact_selected_clusters

    rng = np.random.default_rng(kn)
    B, H, S, D, qn = 1, 3, 4000, 128, 12
    q, k, v, m, qs, ks = _problem(oracle, rng, B, H, H, S, D, qn, kn, density=0.25)
    qt, kt, vt = (to_dev(t[0], dev, torch.bfloat16) for t in (q, k, v))
    mt, qst, kst = to_dev(m[0], dev), to_dev(qs[0], dev), to_dev(ks[0], dev)
    ids, counts = compact_selected_clusters(mt)
    plan_m = plan_block_sparse(mt, qst, kst, S)
    plan_s = plan_block_sparse_from_schedule(ids, counts, qst, kst, S)
    o_m = block_sparse_attention(qt, kt, vt, mt, qst, kst, plan=plan_m)
    o_s = block_sparse_attention(qt, kt, vt, mt, qst, kst, plan=plan_s)
    assert torch.equal(o_m, o_s)
    # through the selector and the drop-in attention call
    from sparsepr_amd.kernels.n8_extension import svg_ear_select_budget_schedule
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    scores = torch.randn((H, qn, kn), device=dev)
    budgets = torch.full((H, qn), S // 5, device=dev, dtype=torch.int32)
    sel_mask, sel_ids, sel_counts = svg_ear_select_budget_schedule(scores, kst, budgets)
    vmap = sel_mask[:, 1:, 1:].contiguous()
    args = (qt[None], kt[None], vt[None], vmap[None], qst[None], kst[None])
    assert torch.equal(dynamic_block_sparse_fwd_flashinfer(*args, is_cpu=False),
                       dynamic_block_sparse_fwd_flashinfer(*args, is_cpu=False,
                                                           selected_schedule=(sel_ids[None], sel_counts[None])))
    # a malformed schedule: shuffled rows with duplicates, -1 and kn entries
    ids_np = np.full((H, qn, kn), -7, np.int32)
    cnt_np = np.zeros((H, qn), np.int32)
    taken = np.zeros((H, qn, kn), bool)
    for h in range(H):
        for i in range(qn):
            row = list(rng.choice(kn, size=rng.integers(0, min(kn, 30) + 1), replace=False))
            row += [-1, kn] + (row[:3] if row else [])
            rng.shuffle(row)
            row = row[:kn]
            ids_np[h, i, :len(row)] = row
            cnt_np[h, i] = len(row) + (2 if i == 0 else 0)  # counts past the listed entries read the -7s
            best = -1
            for c in list(row) + ([-7, -7] if i == 0 else []):
                if 0 <= c < kn and c > best:
                    taken[h, i, c] = True
                best = max(best, c)
    plan_x = plan_block_sparse_from_schedule(to_dev(ids_np, dev), to_dev(cnt_np, dev), qst, kst, S)
    o_x = block_sparse_attention(qt, kt, vt, to_dev(taken, dev), qst, kst, plan=plan_x)
    o_t = block_sparse_attention(qt, kt, vt, to_dev(taken, dev), qst, kst)
    assert torch.equal(o_x, o_t)
    ref, _ = _reference(oracle, q, k, v, taken[None], qs, ks)
    assert np.abs(o_x.float().cpu().numpy() - ref[0]).max() <= 2e-2
