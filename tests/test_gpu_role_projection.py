"""GPU parity: role-coordinate projection + row RMS normalisation against the float64
oracle (TF32-rounded factor), and the full-size unit-RMS property."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

# fp32 sums of 64-128 exact products of O(1) values, normalised to unit RMS
ATOL = 2e-5


@pytest.mark.parametrize("bh,n,d,r", [(2, 1000, 128, 64), (1, 777, 128, 48), (3, 65, 64, 32), (1, 300, 128, 100),
                                      (1, 513, 128, 128), (2, 40, 64, 16)])
def test_role_projection_matches_oracle(dev, oracle, bh, n, d, r):
    from sparsepr_amd.kernels.role_projection import role_projection_rms_triton

    rng = np.random.default_rng(n + r)
    x = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    x[0, min(3, n - 1)] = 0.0
    f = (rng.standard_normal((bh, d, r)) / np.sqrt(d)).astype(np.float32)
    print(f"role projection bh={bh} n={n} d={d} r={r}", flush=True)
    got = role_projection_rms_triton(to_dev(x, dev, torch.bfloat16), to_dev(f, dev))
    torch.cuda.synchronize()
    ref = oracle.role_projection_rms(x, f)
    assert got.shape == (bh, n, r) and got.dtype == torch.float32
    err = np.abs(got.cpu().numpy().astype(np.float64) - ref).max()
    assert err < ATOL, err


def test_role_projection_out_argument_and_errors(dev):
    from sparsepr_amd.kernels.role_projection import role_projection_rms_triton

    x = torch.randn((1, 50, 128), device=dev).to(torch.bfloat16)
    f = torch.randn((1, 128, 64), device=dev)
    out = torch.empty((1, 50, 64), device=dev)
    assert role_projection_rms_triton(x, f, out=out) is out
    with pytest.raises(RuntimeError, match="BLOCK_M"):
        role_projection_rms_triton(x, f, block_m=8)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        role_projection_rms_triton(x, f[:, :64])
    with pytest.raises(RuntimeError, match="output must be"):
        role_projection_rms_triton(x, f, out=torch.empty((1, 50, 63), device=dev))


def test_role_projection_full_size(dev, oracle):
    from sparsepr_amd.kernels.role_projection import role_projection_rms_triton

    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((2, 118800, 128), device=dev, generator=g).to(torch.bfloat16)
    f = torch.randn((2, 128, 64), device=dev, generator=g) / 11.3
    print("role projection full size", flush=True)
    out = role_projection_rms_triton(x, f)
    rms = out.double().pow(2).mean(dim=2).sqrt()
    assert (rms - 1.0).abs().max().item() < 1e-5
    rows = torch.arange(0, 118800, 997, device=dev)
    ref = oracle.role_projection_rms(x[:, rows].float().cpu().numpy(), f.cpu().numpy())
    assert np.abs(out[:, rows].cpu().numpy().astype(np.float64) - ref).max() < ATOL


@pytest.mark.parametrize("bh,n,d,r", [(2, 1000, 128, 64), (3, 4500, 128, 48), (1, 77, 64, 32)])
def test_role_k_projection_matches_oracle(dev, oracle, bh, n, d, r):
    from sparsepr_amd.kernels.role_projection import role_k_projection_normalize

    rng = np.random.default_rng(7 * n + r)
    k = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    f = (rng.standard_normal((bh, d, r)) / np.sqrt(d)).astype(np.float32)
    if bh == 3:
        k[2] = 0.0  # all-zero head: scale 1e-8, key 0
    print(f"role K projection bh={bh} n={n} d={d} r={r}", flush=True)
    kt = to_dev(k, dev, torch.bfloat16)
    key, scale = role_k_projection_normalize(kt, to_dev(f, dev))
    key2, scale2 = role_k_projection_normalize(kt, to_dev(f, dev))
    torch.cuda.synchronize()
    assert torch.equal(key, key2) and torch.equal(scale, scale2)  # deterministic head sums
    ref_key, ref_scale = oracle.role_k_projection_normalize(k, f)
    assert scale.shape == (bh, 1, 1)
    s = scale.cpu().numpy()
    assert np.abs(s - ref_scale).max() <= 1e-5 * np.abs(ref_scale).max()
    assert np.abs(key.cpu().numpy().astype(np.float64) - ref_key).max() < ATOL


def test_role_k_projection_full_size(dev, oracle):
    from sparsepr_amd.kernels.role_projection import role_k_projection_normalize

    g = torch.Generator(device=dev).manual_seed(4)
    k = torch.randn((2, 118800, 128), device=dev, generator=g).to(torch.bfloat16)
    f = torch.randn((2, 128, 64), device=dev, generator=g) / 11.3
    print("role K projection full size", flush=True)
    key, scale = role_k_projection_normalize(k, f)
    # the normalised key has unit RMS over each head
    rms = key.double().pow(2).mean(dim=(1, 2)).sqrt()
    assert (rms - 1.0).abs().max().item() < 1e-5
    rows = torch.arange(0, 118800, 1009, device=dev)
    p = oracle.role_projection_rms(k[:, rows].float().cpu().numpy(), f.cpu().numpy())  # row-normalised
    got = key[:, rows].cpu().numpy().astype(np.float64)
    got_rows = got / np.sqrt((got ** 2).mean(axis=2, keepdims=True))
    assert np.abs(got_rows - p).max() < 1e-4
