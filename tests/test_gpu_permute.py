"""GPU parity: cluster permutation, inverse, concat, row gather/scatter, label argsort.
Bit-exact against the oracle (integer / byte work)."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu


def _labels(rng, rows, n, k):
    return rng.integers(0, k, (rows, n)).astype(np.int32)


@pytest.mark.parametrize("rows,n,k", [(1, 1, 1), (3, 1000, 17), (2, 5000, 512), (1, 70000, 4096), (4, 33, 300)])
def test_argsort_labels_matches_stable_argsort(dev, oracle, rows, n, k):
    from sparsepr_amd.kernels.permute import argsort_labels

    rng = np.random.default_rng(n + k)
    lab = _labels(rng, rows, n, k)
    idx, sizes, offsets = argsort_labels(to_dev(lab, dev), k)
    torch.cuda.synchronize()
    assert (idx.cpu().numpy() == oracle.argsort_labels(lab)).all()
    ref_sizes = np.stack([np.bincount(r, minlength=k) for r in lab])
    assert (sizes.cpu().numpy() == ref_sizes).all()
    ref_off = np.concatenate([np.zeros((rows, 1), np.int64), np.cumsum(ref_sizes, 1)], 1)
    assert (offsets.cpu().numpy() == ref_off).all()


def test_argsort_out_of_range_labels_go_last(dev):
    from sparsepr_amd.kernels.permute import argsort_labels

    lab = np.array([[3, -1, 0, 7, 0, 2]], np.int32)  # k = 4: -1 and 7 are out of range
    idx, sizes, offsets = argsort_labels(to_dev(lab, dev), 4)
    assert idx.cpu().tolist() == [[2, 4, 5, 0, 1, 3]]
    assert sizes.cpu().tolist() == [[2, 0, 1, 1]]
    assert offsets.cpu().tolist() == [[0, 2, 2, 3, 4]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 2, 1000, 128), (2, 3, 257, 64), (1, 1, 5, 3)])
def test_permute_and_inverse_bit_exact(dev, oracle, dtype, shape):
    from sparsepr_amd.kernels.permute import (apply_inverse_permutation_triton,
                                              permute_tensor_by_labels_triton)

    B, H, S, D = shape
    rng = np.random.default_rng(S * D)
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dtype).to(dev)
    lab = _labels(rng, B * H, S, 11)
    y, idx = permute_tensor_by_labels_triton(x, to_dev(lab, dev), dim=2)
    ref_idx = oracle.argsort_labels(lab)
    assert idx.dtype == torch.int32 and (idx.cpu().numpy() == ref_idx).all()
    xc = x.reshape(B * H, S, D).cpu()
    ref = xc[torch.arange(B * H)[:, None], torch.from_numpy(ref_idx).long()]
    assert torch.equal(y.reshape(B * H, S, D).cpu(), ref)
    back = apply_inverse_permutation_triton(y, idx, dim=2)
    assert torch.equal(back.cpu(), x.cpu())
    # explicit sorted_indices path
    y2, _ = permute_tensor_by_labels_triton(x, None, dim=2, sorted_indices=idx)
    assert torch.equal(y2, y)


def test_permute_concatenated(dev, oracle):
    from sparsepr_amd.kernels.permute import permute_concatenated_tensors_by_labels_triton

    rng = np.random.default_rng(5)
    pre = torch.randn(1, 3, 300, 128, dtype=torch.bfloat16, device=dev)
    suf = torch.randn(1, 3, 17, 128, dtype=torch.bfloat16, device=dev)
    lab = _labels(rng, 3, 317, 9)
    out, idx = permute_concatenated_tensors_by_labels_triton(pre, suf, to_dev(lab, dev), dim=2)
    full = torch.cat([pre, suf], 2).reshape(3, 317, 128).cpu()
    ref = full[torch.arange(3)[:, None], torch.from_numpy(oracle.argsort_labels(lab)).long()]
    assert torch.equal(out.reshape(3, 317, 128).cpu(), ref)
    with pytest.raises(RuntimeError):
        permute_concatenated_tensors_by_labels_triton(pre, suf[..., :64], to_dev(lab, dev), dim=2)


def test_gather_scatter_rows_and_bounds(dev):
    from sparsepr_amd import _lib
    from sparsepr_amd.flash_kmeans.kmeans_impl import gather_rows

    src = torch.arange(2 * 10 * 8, dtype=torch.float32, device=dev).reshape(2, 10, 8)
    idx = torch.tensor([[9, 0, 3], [1, 1, 12]], dtype=torch.int32, device=dev)  # 12 is out of range
    g = gather_rows(src, idx)
    assert torch.equal(g[0, 0], src[0, 9]) and torch.equal(g[1, 1], src[1, 1])
    assert (g[1, 2] == 0).all()
    dst = torch.full((2, 10, 8), -1.0, device=dev)
    _lib.call("spr_scatter_rows", g.data_ptr(), 3, idx.data_ptr(), dst.data_ptr(), 10, 2, 32, _lib.stream(dev))
    assert torch.equal(dst[0, 3], src[0, 3]) and (dst[0, 5] == -1).all()
    assert torch.equal(dst[1, 1], src[1, 1])


def test_permute_full_size_round_trip(dev):
    """BASELINE HunyuanVideo shape: 24 x 118,800 x 128 bf16 — size-independent properties."""
    from sparsepr_amd.kernels.permute import (apply_inverse_permutation_triton, argsort_labels,
                                              permute_tensor_by_labels_triton)

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(1, 24, 118800, 128, dtype=torch.bfloat16, device=dev, generator=g)
    lab = torch.randint(0, 512, (24, 118800), dtype=torch.int32, device=dev, generator=g)
    y, idx = permute_tensor_by_labels_triton(x, lab, dim=2)
    sl = torch.gather(lab, 1, idx.long())
    assert bool((sl[:, 1:] >= sl[:, :-1]).all())
    same = sl[:, 1:] == sl[:, :-1]
    assert bool((idx[:, 1:][same] > idx[:, :-1][same]).all())  # stable
    assert torch.equal(apply_inverse_permutation_triton(y, idx, dim=2), x)
    _, sizes, offsets = argsort_labels(lab, 512)
    assert torch.equal(sizes.sum(1), torch.full((24,), 118800, dtype=torch.int64, device=dev).to(sizes.dtype))


def test_inverse_permutation_of_a_row_slice_in_place(dev):
    """The video rows of a longer [B, H, S + T, D] tensor (a slice, not packed) are
    un-permuted in place: the same bits as from a packed copy, and a round trip."""
    from sparsepr_amd.kernels.permute import apply_inverse_permutation_triton, permute_tensor_by_labels_triton

    g = torch.Generator(device=dev).manual_seed(11)
    B, H, S, T, D = 2, 3, 1000, 77, 128
    full = torch.randn((B, H, S + T, D), device=dev, generator=g).to(torch.bfloat16)
    idx = torch.argsort(torch.rand((B * H, S), device=dev, generator=g), dim=-1).to(torch.int32)
    view = full[:, :, :S]
    assert not view.is_contiguous()
    got = apply_inverse_permutation_triton(view, idx, dim=2)
    ref = apply_inverse_permutation_triton(view.contiguous(), idx, dim=2)
    assert torch.equal(got, ref)
    back, _ = permute_tensor_by_labels_triton(got, None, 2, sorted_indices=idx)
    assert torch.equal(back, view)


def test_inverse_permutation_of_an_expanded_tensor(dev):
    """An expanded tensor (zero head strides: every head views one [S, D] block) takes the
    copying path, not the in-place one: each head is un-permuted from the shared block.  The
    strided entry point refuses a head stride below S rows."""
    from sparsepr_amd import _lib
    from sparsepr_amd.kernels.permute import apply_inverse_permutation_triton

    g = torch.Generator(device=dev).manual_seed(12)
    B, H, S, D = 2, 3, 500, 128
    block = torch.randn((1, 1, S, D), device=dev, generator=g).to(torch.bfloat16)
    view = block.expand(B, H, S, D)
    assert view.stride(0) == 0 and view.stride(1) == 0
    idx = torch.argsort(torch.rand((B * H, S), device=dev, generator=g), dim=-1).to(torch.int32)
    got = apply_inverse_permutation_triton(view, idx, dim=2)
    ref = apply_inverse_permutation_triton(view.contiguous(), idx, dim=2)
    assert torch.equal(got, ref)
    out = torch.empty((B * H, S, D), device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head stride"):
        _lib.call("spr_inverse_permute_rows_strided", _lib.ptr(block), 0, _lib.ptr(idx), _lib.ptr(out), B * H, S,
                  D * 2, _lib.stream(dev))
