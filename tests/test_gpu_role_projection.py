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
                                      (1, 513, 128, 128), (2, 40, 64, 16), (24, 30001, 128, 64)])
def test_role_projection_matches_oracle(dev, oracle, bh, n, d, r):
    """(24, 30001, 128, 64): 118 blocks of 256 tokens per head against about 1,000 resident
    workgroups, so workgroups walk several blocks of their head (and a short last one)."""
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


@pytest.mark.parametrize("bh,n,d,r", [(2, 1000, 128, 64), (3, 4500, 128, 48), (1, 77, 64, 32), (24, 60001, 128, 48)])
def test_role_k_projection_matches_oracle(dev, oracle, bh, n, d, r):
    """(24, 60001, 128, 48): 59 blocks of 1024 tokens per head in the sum pass and 235 of 256
    in the scaling pass, against about 1,000 resident workgroups, so workgroups walk several
    blocks of their head (and a short last one) in both."""
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


@pytest.mark.parametrize("precision", ["high", "highest", "medium"])
def test_role_k_projection_precisions(dev, oracle, precision):
    """The K projection under role_kv_matmul_precision (n8_v6.py:77-86): the factor as TF32
    ("high"), fp32 ("highest", three exact bf16 pieces) or bf16 ("medium") against the float64
    oracle on the same operand rounding; the three differ from one another by more than the
    tolerance, so each rounding is what is checked."""
    from sparsepr_amd.kernels.role_projection import role_k_projection_normalize

    rng = np.random.default_rng(31)
    bh, n, d, r = 2, 3000, 128, 48
    k = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    f = (rng.standard_normal((bh, d, r)) / np.sqrt(d)).astype(np.float32)
    key, scale = role_k_projection_normalize(to_dev(k, dev, torch.bfloat16), to_dev(f, dev), precision=precision)
    torch.cuda.synchronize()
    got = key.cpu().numpy().astype(np.float64)
    refs = {p: oracle.role_k_projection_normalize(k, f, p)[0].astype(np.float64) for p in ("high", "highest", "medium")}
    assert np.abs(got - refs[precision]).max() < ATOL
    for other, ref in refs.items():
        if other != precision:
            assert np.abs(got - ref).max() > 4 * ATOL
    assert np.abs(scale.cpu().numpy() - oracle.role_k_projection_normalize(k, f, precision)[1]).max() <= 1e-5


@pytest.mark.parametrize("precision", ["high", "highest", "medium"])
def test_role_kv_projection_and_init(dev, oracle, precision):
    """Joint K/V role features (_role_kv_projection_normalize_fp32, n8_v6.py:91-103): K features
    in the first R_k columns, (v_weight value) / value_scale in the next R_v; the warm start
    (_role_kv_init_projection_fp32, :118-126) through the strided, weighted row projection."""
    from sparsepr_amd.kernels.role_metric import project_rows
    from sparsepr_amd.kernels.role_projection import role_kv_projection_normalize

    rng = np.random.default_rng(32)
    bh, n, d, rk, rv, w, c = 2, 2500, 128, 48, 16, 0.35, 70
    k = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((bh, n, d)).astype(np.float32))
    kf = (rng.standard_normal((bh, d, rk)) / np.sqrt(d)).astype(np.float32)
    vf = (rng.standard_normal((bh, d, rv)) / np.sqrt(d)).astype(np.float32)
    feats, ks, vs = role_kv_projection_normalize(to_dev(k, dev, torch.bfloat16), to_dev(v, dev, torch.bfloat16),
                                                 to_dev(kf, dev), to_dev(vf, dev), w, precision=precision)
    rfeat, rks, rvs = oracle.role_kv_projection_normalize(k, v, kf, vf, w, precision)
    assert feats.shape == (bh, n, rk + rv)
    assert np.abs(feats.cpu().numpy().astype(np.float64) - rfeat).max() < ATOL
    assert np.abs(ks.cpu().numpy() - rks).max() <= 1e-5 and np.abs(vs.cpu().numpy() - rvs).max() <= 1e-5
    kc = rng.standard_normal((bh, c, d)).astype(np.float32)
    vc = rng.standard_normal((bh, c, d)).astype(np.float32)
    init = torch.full((bh, c, rk + rv), 7.0, device=dev)
    project_rows(to_dev(kc, dev), to_dev(kf, dev), divisor=ks, precision=precision, out=init)
    project_rows(to_dev(vc, dev), to_dev(vf, dev), divisor=vs, precision=precision, weight=w, out=init, out_col=rk)
    ref_init = np.concatenate((oracle.project_rows(kc, kf, rks.reshape(-1), precision=precision),
                               oracle.project_rows(vc, vf, rvs.reshape(-1), precision=precision, weight=w)), axis=2)
    assert np.abs(init.cpu().numpy() - ref_init).max() <= 1e-4 * np.abs(ref_init).max()
