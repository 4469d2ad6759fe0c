"""GPU parity: SVG-EAR routing scores (value error with and without the Jensen term,
grouped, attention mass) against the float64 oracle, and full-size properties."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

# Scores are logs of fp32 sums of exponentials of fp32 MFMA logits; the oracle is float64
# with the final max.  2e-3 in log space is 0.2 % of the value-error sum; a dropped term,
# a sign error or a wrong token run moves a score by far more.
ATOL = 2e-3


def _case(seed, qh, group, qn, sizes, extra=5, d=128, qscale=0.4):
    rng = np.random.default_rng(seed)
    kvh = qh // group
    kn = sizes.shape[1]
    t = int(sizes.sum(axis=1).max()) + extra
    qc = (rng.standard_normal((qh, qn, d)) * qscale).astype(np.float32)
    k = rng.standard_normal((kvh, t, d)).astype(np.float32)
    v = rng.standard_normal((kvh, t, d)).astype(np.float32)
    kc = (rng.standard_normal((kvh, kn, d)) * 0.5).astype(np.float32)
    vc = (rng.standard_normal((kvh, kn, d)) * 0.5).astype(np.float32)
    var = rng.uniform(0.0, 1.5, (kvh, kn, d)).astype(np.float32)
    return qc, k, v, kc, vc, var


def _bf16_np(oracle, x):
    return oracle.to_bf16(x)


def _check(got, ref):
    got = got.cpu().numpy().astype(np.float64)
    ref = ref.astype(np.float64)
    assert (np.isneginf(got) == np.isneginf(ref)).all()
    assert np.isfinite(got[~np.isneginf(ref)]).all()
    fin = np.isfinite(ref)
    if fin.any():
        err = np.abs(got[fin] - ref[fin]).max()
        assert err < ATOL, err


SIZES = [
    np.array([[0, 1, 31, 32, 33, 64, 100, 7, 250]], np.int32),
    np.array([[5, 0, 40], [70, 3, 0]], np.int32),
]


@pytest.mark.parametrize("qh,group,qn,si", [(1, 1, 128, 0), (2, 2, 40, 0), (2, 1, 200, 1), (4, 2, 33, 1)])
@pytest.mark.parametrize("jensen", [0.0, 0.3])
def test_value_error_scores_match_oracle(dev, oracle, qh, group, qn, si, jensen):
    from sparsepr_amd.kernels.svg_ear import svg_ear_value_error_scores_triton

    sizes = SIZES[si]
    if sizes.shape[0] != qh // group:
        sizes = np.repeat(sizes[:1], qh // group, axis=0)
    qc, k, v, kc, vc, var = _case(qh * 100 + qn, qh, group, qn, sizes)
    k, v = _bf16_np(oracle, k), _bf16_np(oracle, v)
    print(f"value error qh={qh} group={group} qn={qn} sizes={sizes.tolist()} jensen={jensen}", flush=True)
    got = svg_ear_value_error_scores_triton(
        qcentroids=to_dev(qc, dev), k_sorted=to_dev(k, dev, torch.bfloat16), v_sorted=to_dev(v, dev, torch.bfloat16),
        kcentroids=to_dev(kc, dev), vcentroids=to_dev(vc, dev), kcluster_sizes=to_dev(sizes, dev),
        gqa_group=group, var_k_diag=to_dev(var, dev) if jensen > 0 else None, jensen_var_cap=jensen)
    torch.cuda.synchronize()
    ref = oracle.svg_ear_value_error_scores(qc, k, v, kc, vc, sizes, group, var if jensen > 0 else None, jensen)
    _check(got, ref)


@pytest.mark.parametrize("qh,group,qn,si", [(1, 1, 128, 0), (4, 2, 70, 1), (2, 1, 300, 0)])
def test_attention_mass_scores_match_oracle(dev, oracle, qh, group, qn, si):
    from sparsepr_amd.kernels.svg_ear import attention_mass_scores_triton

    sizes = SIZES[si]
    if sizes.shape[0] != qh // group:
        sizes = np.repeat(sizes[:1], qh // group, axis=0)
    qc, k, _, _, _, _ = _case(qh * 7 + qn, qh, group, qn, sizes, qscale=1.5)
    k = _bf16_np(oracle, k)
    print(f"attention mass qh={qh} group={group} qn={qn}", flush=True)
    got = attention_mass_scores_triton(qcentroids=to_dev(qc, dev), k_sorted=to_dev(k, dev, torch.bfloat16),
                                       kcluster_sizes=to_dev(sizes, dev), gqa_group=group)
    torch.cuda.synchronize()
    _check(got, oracle.attention_mass_scores(qc, k, sizes, group))


def test_grouped_scores_equal_ungrouped(dev, oracle):
    from sparsepr_amd.kernels.svg_ear import (svg_ear_grouped_value_error_scores_triton,
                                              svg_ear_value_error_scores_triton)

    sizes = np.array([[10, 0, 45, 3], [1, 60, 2, 0]], np.int32)
    qc, k, v, kc, vc, _ = _case(5, 8, 4, 50, sizes)
    args = dict(qcentroids=to_dev(qc, dev), k_sorted=to_dev(k, dev, torch.bfloat16),
                v_sorted=to_dev(v, dev, torch.bfloat16), kcentroids=to_dev(kc, dev), vcentroids=to_dev(vc, dev),
                kcluster_sizes=to_dev(sizes, dev), gqa_group=4)
    a = svg_ear_grouped_value_error_scores_triton(**args)
    b = svg_ear_value_error_scores_triton(**args)
    assert torch.equal(a, b)


def test_validation_errors(dev):
    from sparsepr_amd.kernels.svg_ear import attention_mass_scores_triton, svg_ear_value_error_scores_triton

    qc = torch.zeros((2, 4, 64), device=dev)
    k = torch.zeros((2, 10, 64), device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="DIM=128"):
        attention_mass_scores_triton(qcentroids=qc, k_sorted=k, kcluster_sizes=torch.ones((2, 3), device=dev),
                                     gqa_group=1)
    qc = torch.zeros((2, 4, 128), device=dev)
    k = torch.zeros((1, 10, 128), device=dev, dtype=torch.bfloat16)
    kc = torch.zeros((1, 3, 128), device=dev)
    with pytest.raises(RuntimeError, match="GQA mismatch"):
        svg_ear_value_error_scores_triton(qcentroids=qc, k_sorted=k, v_sorted=k, kcentroids=kc, vcentroids=kc,
                                          kcluster_sizes=torch.ones((1, 3), device=dev), gqa_group=1)
    with pytest.raises(RuntimeError, match="requires var_k_diag"):
        svg_ear_value_error_scores_triton(qcentroids=qc, k_sorted=k, v_sorted=k, kcentroids=kc, vcentroids=kc,
                                          kcluster_sizes=torch.ones((1, 3), device=dev), gqa_group=2,
                                          jensen_var_cap=0.5)
    with pytest.raises(RuntimeError, match="BQ="):
        svg_ear_value_error_scores_triton(qcentroids=qc, k_sorted=k, v_sorted=k, kcentroids=kc, vcentroids=kc,
                                          kcluster_sizes=torch.ones((1, 3), device=dev), gqa_group=2, block_q=12)


def _full_problem(dev, seed, tokens=118800, kn=512, qn=128):
    g = torch.Generator(device=dev).manual_seed(seed)
    sizes = torch.randint(0, 2 * tokens // kn, (1, kn), device=dev, generator=g, dtype=torch.int32)
    sizes[0, ::37] = 0
    over = int(sizes.sum()) - tokens
    while over > 0:  # trim to the token count
        i = int(torch.argmax(sizes))
        cut = min(over, int(sizes[0, i]) - 1)
        sizes[0, i] -= cut
        over -= cut
    k = torch.randn((1, tokens, 128), device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn((1, tokens, 128), device=dev, generator=g).to(torch.bfloat16)
    qc = torch.randn((1, qn, 128), device=dev, generator=g) * 0.7
    kc = torch.randn((1, kn, 128), device=dev, generator=g) * 0.3
    vc = torch.randn((1, kn, 128), device=dev, generator=g) * 0.3
    return sizes, k, v, qc, kc, vc


def test_full_size_mass_sums_to_total_logsumexp(dev, oracle):
    """Size-independent identity at the C4 token count: the log-sum-exp over clusters of
    the mass scores is the log-sum-exp of every token's logit."""
    from sparsepr_amd.kernels.svg_ear import attention_mass_scores_triton

    sizes, k, _, qc, _, _ = _full_problem(dev, 0)
    print("full-size attention mass", flush=True)
    scores = attention_mass_scores_triton(qcentroids=qc, k_sorted=k, kcluster_sizes=sizes, gqa_group=1)
    used = int(sizes.sum())
    qt = torch.from_numpy(oracle.tf32_rna(qc.cpu().numpy())).to(dev).double()
    logits = (qt[0] @ k[0, :used].double().T) * float(np.float32(1.0) / np.sqrt(np.float32(128)))
    want = torch.logsumexp(logits, dim=1)
    got = torch.logsumexp(scores[0].double(), dim=1)
    assert torch.isneginf(scores[0, :, sizes[0] == 0]).all()
    assert (got - want).abs().max().item() < ATOL


def test_full_size_value_error_sampled_clusters(dev, oracle):
    """C4 token count and cluster count; a sample of clusters re-scored by the oracle."""
    from sparsepr_amd.kernels.svg_ear import svg_ear_value_error_scores_triton

    sizes, k, v, qc, kc, vc = _full_problem(dev, 1)
    print("full-size value error", flush=True)
    scores = svg_ear_value_error_scores_triton(qcentroids=qc, k_sorted=k, v_sorted=v, kcentroids=kc, vcentroids=vc,
                                               kcluster_sizes=sizes, gqa_group=1).cpu().numpy()
    s = sizes[0].cpu().numpy()
    off = np.concatenate(([0], np.cumsum(s)))
    kk, vv = k[0].float().cpu().numpy(), v[0].float().cpu().numpy()
    q_np, kc_np, vc_np = qc.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()
    for c in list(np.nonzero(s)[0][::41]) + [int(np.argmax(s))]:
        ref = oracle.svg_ear_value_error_scores(q_np, kk[None, off[c]:off[c + 1]], vv[None, off[c]:off[c + 1]],
                                                kc_np[:, c:c + 1], vc_np[:, c:c + 1], s[None, c:c + 1], 1)
        err = np.abs(scores[0, :, c].astype(np.float64) - ref[0, :, 0]).max()
        assert err < ATOL, (c, err)
    assert np.isneginf(scores[0][:, s == 0]).all()


@pytest.mark.parametrize("reformulation,block_k,sparse_bf16", [("skipped", 32, True), ("n3_residual", 32, False),
                                                               ("skipped", 16, False), ("n3_residual", 16, True)])
def test_svg_ear_compensation(dev, oracle, reformulation, block_k, sparse_bf16):
    """svg_ear_compensation_triton (svg_ear.py:289-369, :603-678) against the float64
    restatement on the same inputs: 70 key clusters (a partial last block), empty clusters,
    a random selection map, bf16 queries; max-abs within 2e-3 of the largest output (the
    TF32 rounding of an fp32 weight can land one step from the float64 one's); the NaN of a
    row with LSE -inf whose first block adds nothing is reproduced."""
    from sparsepr_amd.kernels.svg_ear import svg_ear_compensation_triton

    rng = np.random.default_rng(block_k + len(reformulation))
    bh, t, d, kn, qn = 3, 700, 128, 70, 12
    q = oracle.to_bf16(rng.standard_normal((bh, t, d)).astype(np.float32))
    sparse = rng.standard_normal((bh, t, d)).astype(np.float32) * 0.3
    if sparse_bf16:
        sparse = oracle.to_bf16(sparse)
    lse = (rng.standard_normal((bh, t)) * 2.0).astype(np.float32)
    labels = rng.integers(0, qn, (bh, t)).astype(np.int64)
    dmap = rng.random((bh, qn + 1, kn + 1)) < 0.35
    kc = (rng.standard_normal((bh, kn, d)) * 0.5).astype(np.float32)
    vc = rng.standard_normal((bh, kn, d)).astype(np.float32)
    counts = rng.integers(0, 40, (bh, kn)).astype(np.float32)
    counts[:, ::9] = 0.0
    # a row with LSE -inf whose first block adds nothing (skipped: its label row selects the
    # whole block; n3_residual: the block's clusters of that head are empty): NaN in both
    lse[1, 7] = -np.inf
    if reformulation == "skipped":
        dmap[1, labels[1, 7] + 1, 1:block_k + 1] = True
    else:
        counts[1, :block_k] = 0.0
    out = svg_ear_compensation_triton(
        q_flat=to_dev(q, dev, torch.bfloat16), sparse_flat=to_dev(sparse, dev, torch.bfloat16 if sparse_bf16 else None),
        lse_flat=to_dev(lse, dev), qlabels_gen=to_dev(labels, dev), dynamic_map_query=to_dev(dmap, dev),
        kcentroids=to_dev(kc, dev), kcluster_sizes=to_dev(counts.astype(np.int64), dev), vcentroids=to_dev(vc, dev),
        reformulation=reformulation, block_k=block_k)
    ref = oracle.svg_ear_compensation(q, sparse, lse, labels, dmap, kc, counts, vc, reformulation, block_k)
    got = out.cpu().numpy()
    assert (np.isnan(got) == np.isnan(ref)).all() and np.isnan(ref[1, 7]).all()
    fin = ~np.isnan(ref)
    assert np.abs(got[fin] - ref[fin]).max() <= 2e-3 * np.abs(ref[fin]).max()
    with pytest.raises(RuntimeError, match="reformulation"):
        svg_ear_compensation_triton(q_flat=out, sparse_flat=out, lse_flat=to_dev(lse, dev),
                                    qlabels_gen=to_dev(labels, dev), dynamic_map_query=to_dev(dmap, dev),
                                    kcentroids=to_dev(kc, dev), kcluster_sizes=to_dev(counts, dev),
                                    vcentroids=to_dev(vc, dev), reformulation="bogus")
