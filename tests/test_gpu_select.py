"""GPU parity: top-p cluster-pair map (bit-exact, canonical fp32 order), budget
selector (reference KAT + random, both semantics), compaction, density."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _centroids(rng, bh, qn, kn, d, scale=1.0):
    qc = (rng.standard_normal((bh, qn, d)) * scale).astype(np.float32)
    kc = (rng.standard_normal((bh, kn, d)) * scale).astype(np.float32)
    ks = rng.integers(0, 400, (bh, kn)).astype(np.int32)
    ks[:, ::7] = 0  # empty clusters
    return qc, kc, ks


# key-cluster counts that reach every register width of the one-wave sort (1 .. 64 keys per
# lane: kn up to 64, 128, 256, 512, 1024, 2048, 4096)
@pytest.mark.parametrize("bh,qn,kn,d", [(2, 3, 1, 64), (2, 5, 2, 64), (4, 32, 64, 64), (2, 9, 100, 64), (2, 17, 256, 64),
                                        (2, 128, 512, 128),
                                        (1, 5, 300, 128), (1, 11, 1000, 128), (1, 3, 2000, 64),
                                        (1, 3, 4096, 64), (3, 100, 500, 128)])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("p,ratio", [(0.9, 0.0), (0.7, 0.0), (0.95, 0.1)])
def test_topp_map_bit_exact(dev, oracle, bh, qn, kn, d, bf16, p, ratio):
    from sparsepr_amd.kmeans_utils import identify_dynamic_map

    rng = np.random.default_rng(bh * 1000 + kn + int(bf16))
    qc, kc, ks = _centroids(rng, bh, qn, kn, d, scale=0.4)
    if bf16:
        qc, kc = oracle.to_bf16(qc), oracle.to_bf16(kc)
    dt = torch.bfloat16 if bf16 else torch.float32
    qs = np.full((bh, qn), 10, np.int32)
    got = identify_dynamic_map(to_dev(qc, dev, dt)[None], to_dev(kc, dev, dt)[None], to_dev(qs, dev)[None],
                               to_dev(ks, dev)[None], p, ratio)
    ref = oracle.identify_dynamic_map(qc, kc, ks, p, ratio, bf16=bf16)
    assert got.dtype == torch.bool
    assert (got[0].cpu().numpy() == ref).all()


@pytest.mark.parametrize("bh,qn,kn,d", [(4, 32, 64, 64), (2, 128, 512, 128), (3, 100, 500, 128)])
@pytest.mark.parametrize("p", [0.5, 0.85, 0.95])
def test_top_p_key_budgets_exact(dev, oracle, bh, qn, kn, d, p):
    """SVG2 key-token budgets (n8_v6.py:181-230): integers, equal to the oracle's."""
    from sparsepr_amd.kernels.selection import top_p_key_budgets

    rng = np.random.default_rng(bh * 7 + kn + int(100 * p))
    qc, kc, ks = _centroids(rng, bh, qn, kn, d, scale=0.4)
    got = top_p_key_budgets(to_dev(qc, dev), to_dev(kc, dev), to_dev(ks, dev), p)
    assert got.dtype == torch.int64 and tuple(got.shape) == (bh, qn)
    assert (got.cpu().numpy() == oracle.svg_top_p_key_budgets(qc, kc, ks, p)).all()
    with pytest.raises(ValueError, match="svg_ear_top_p"):
        top_p_key_budgets(to_dev(qc, dev), to_dev(kc, dev), to_dev(ks, dev), 1.5)


def test_topp_map_all_empty_keeps_everything(dev, oracle):
    from sparsepr_amd.kmeans_utils import identify_dynamic_map

    qc = np.ones((1, 2, 8), np.float32)
    kc = np.ones((1, 5, 8), np.float32)
    ks = np.zeros((1, 5), np.int32)
    got = identify_dynamic_map(to_dev(qc, dev)[None], to_dev(kc, dev)[None], None, to_dev(ks, dev)[None], 0.9)
    assert got.all()
    assert (oracle.identify_dynamic_map(qc, kc, ks, 0.9) == got[0].cpu().numpy()).all()


def test_topp_map_full_size_invariants(dev, oracle):
    """HunyuanVideo routing shape: 24 heads x 128 q-clusters x 512 k-clusters, D=128."""
    from sparsepr_amd.kmeans_utils import density_calculation, identify_dynamic_map

    g = torch.Generator(device=dev)
    g.manual_seed(1)
    qc = (0.3 * torch.randn(1, 24, 128, 128, device=dev, generator=g)).to(torch.bfloat16)
    kc = (0.3 * torch.randn(1, 24, 512, 128, device=dev, generator=g)).to(torch.bfloat16)
    ks = torch.randint(0, 500, (1, 24, 512), device=dev, generator=g, dtype=torch.int32)
    qs = torch.randint(1, 1000, (1, 24, 128), device=dev, generator=g, dtype=torch.int32)
    m = identify_dynamic_map(qc, kc, qs, ks, 0.9)
    assert bool((m.sum(-1) >= 1).all())
    ref = oracle.identify_dynamic_map(qc[0].float().cpu().numpy(), kc[0].float().cpu().numpy(),
                                      ks[0].cpu().numpy(), 0.9, bf16=True)
    assert (m[0].cpu().numpy() == ref).all()
    dens = density_calculation(m, qs, ks)
    ref_d = oracle.density(ref[None], qs.cpu().numpy(), ks.cpu().numpy())
    assert np.allclose(dens.cpu().numpy(), ref_d, rtol=1e-6)


@pytest.mark.parametrize("qn,kn", [(7, 37), (5, 48)])
def test_density_byte_and_vector_paths(dev, oracle, qn, kn):
    """density_calculation on maps whose rows are not (37) and are (48) whole 16-byte
    vectors, against the oracle's closed form."""
    from sparsepr_amd.kmeans_utils import density_calculation

    rng = np.random.default_rng(qn * kn)
    m = rng.random((3, qn, kn)) < 0.3
    qs = rng.integers(0, 900, (3, qn)).astype(np.int32)
    ks = rng.integers(0, 400, (3, kn)).astype(np.int32)
    got = density_calculation(to_dev(m, dev)[None], to_dev(qs, dev)[None], to_dev(ks, dev)[None])
    ref = oracle.density(m[None], qs[None], ks[None])
    assert np.allclose(got.cpu().numpy(), ref, rtol=1e-6)


def test_selector_known_answer_gpu(dev):
    from sparsepr_amd.kernels.n8_extension import (compact_selected_clusters, load_n8_kernels,
                                                   svg_ear_select_budget_schedule)
    from sparsepr_amd.kernels.selector_budget import exact_budget_dynamic_map_triton

    kat = json.loads((GOLDEN / "selector_kat.json").read_text())
    scores = torch.tensor(kat["scores"], device=dev)
    sizes = torch.tensor(kat["sizes"], device=dev, dtype=torch.int32)
    budgets = torch.tensor(kat["budgets"], device=dev, dtype=torch.int32)
    block_map, ids, counts = svg_ear_select_budget_schedule(scores, sizes, budgets)
    expected = torch.tensor(kat["expected_mask"], device=dev)
    assert torch.equal(block_map[0, 1:, 1:], expected)
    assert block_map[0, 0, 0].item() and block_map[0, 1:, 0].all().item()
    assert counts.cpu().tolist() == kat["expected_counts"]
    assert ids[0, 0, :3].cpu().tolist() == kat["expected_ids"][0][0]
    assert ids[0, 1, :2].cpu().tolist() == kat["expected_ids"][0][1]
    cids, ccounts = compact_selected_clusters(expected)
    assert ccounts.cpu().tolist() == kat["expected_counts"][0]
    assert cids[0, :3].cpu().tolist() == [0, 1, 2] and cids[1, :2].cpu().tolist() == [1, 2]
    tri = exact_budget_dynamic_map_triton(scores, sizes, budgets)
    assert torch.equal(tri, block_map)
    mod = load_n8_kernels(required=True)
    assert hasattr(mod, "svg_ear_select_budget_schedule") and hasattr(mod, "compact_selected_clusters")


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("bh,qn,kn", [(2, 3, 1), (2, 5, 2), (2, 7, 9), (1, 3, 64), (1, 3, 65), (2, 9, 100), (2, 17, 200), (3, 50, 512),
                                     (3, 100, 1000), (1, 6, 2000), (1, 4, 4096)])
def test_selector_random_vs_oracle(dev, oracle, mode, bh, qn, kn):
    """Rows of every register width of the one-wave sort (kn up to 64 E for E = 1 .. 64), with
    many tied scores (the index breaks them) and empty clusters."""
    from sparsepr_amd.kernels.selection import select_budget

    rng = np.random.default_rng(mode * 7 + kn)
    scores = rng.integers(-5, 6, (bh, qn, kn)).astype(np.float32)  # many ties
    scores[..., ::3] = rng.standard_normal(scores[..., ::3].shape)
    scores[..., 1::11] = -0.0  # ties with the +0.0 entries: compared as equal, so the index decides
    scores[..., 2::13] = -np.inf  # empty-cluster scores
    sizes = rng.integers(0, 50, (bh, kn)).astype(np.int32)
    budgets = rng.integers(0, 25 * kn, (bh, qn)).astype(np.int32)
    out, ids, counts = select_budget(to_dev(scores, dev), to_dev(sizes, dev), to_dev(budgets, dev), mode,
                                     with_schedule=True)
    ref = oracle.select_budget(scores, sizes, budgets, mode)
    assert (out.cpu().numpy() == ref).all()
    rids, rcounts = oracle.compact_selected_clusters(ref[:, 1:, 1:])
    assert (counts.cpu().numpy() == rcounts).all()
    ids_np = ids.cpu().numpy()
    for h in range(bh):
        for q in range(qn):
            c = rcounts[h, q]
            assert (ids_np[h, q, :c] == rids[h, q, :c]).all()


def test_compaction_random(dev, oracle):
    from sparsepr_amd.kernels.n8_extension import compact_selected_clusters

    rng = np.random.default_rng(3)
    m = rng.random((5, 6, 777)) < 0.3
    ids, counts = compact_selected_clusters(to_dev(m, dev))
    rids, rcounts = oracle.compact_selected_clusters(m)
    assert (counts.cpu().numpy() == rcounts).all()
    for idx in np.ndindex(5, 6):
        c = rcounts[idx]
        assert (ids.cpu().numpy()[idx][:c] == rids[idx][:c]).all()
