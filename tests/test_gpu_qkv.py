"""GPU parity of the model-edge fusions (Wan and Cosmos2.5 Q/K RMSNorm + RoPE + layout)
against the float64 oracle with the same rounding points.

Tolerance: the kernel evaluates (x * inv) * w and the rotation in fp32 before each of the
two roundings to the model dtype, the oracle in float64; a value on a rounding boundary can
round one way in one and the other way in the other.  An output ulp is at most 2u |out|; a
flip of the normalised inputs r0, r1 (at most 2u |r| each) moves r0 cos - r1 sin by at most
2u |pair| (Cauchy-Schwarz; a rotation keeps the pair's norm).  Bound:
|got - ref| <= (2u + 1e-6)(|ref| + |pair|), u = 2^-8 (bf16), 2^-11 (fp16), 2^-24 (fp32), the
1e-6 covering the fp32 chain and sincosf.  V is moved, not computed: exact."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu

UNIT = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}
NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _model_values(rng, shape, dtype, scale=1.0):
    x = (scale * rng.standard_normal(shape)).astype(np.float32)
    return torch.from_numpy(x).to(dtype).float().numpy()  # representable in the dtype


def _check(got, ref, pair_mag, dtype, exact_share):
    got = got.float().cpu().numpy().astype(np.float64)
    u = UNIT[dtype]
    err = np.abs(got - ref)
    bound = (2 * u + 1e-6) * (np.abs(ref) + pair_mag) + 1e-30
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert (err <= bound).all(), (worst, got[worst], ref[worst], pair_mag[worst])
    assert np.mean(err == 0) >= exact_share


_WAN_CASES = [(torch.bfloat16, (2, 300, 4, 128)), (torch.float16, (2, 300, 4, 128)),
              (torch.float32, (2, 300, 4, 128)), (torch.bfloat16, (1, 130, 20, 128)),
              (torch.bfloat16, (1, 70, 40, 128)), (torch.bfloat16, (1, 50, 3, 100)),
              (torch.bfloat16, (1, 20, 72, 128))]


@pytest.mark.parametrize("dtype,shape", _WAN_CASES)
def test_wan_qkv_norm_rope_layout(dev, oracle, dtype, shape):
    """Vector paths with 1, 2 and 4 vectors per thread (C = 512, 2560, 5120) in bf16, fp16
    and fp32, the pair path (D = 100) and C > 8192 (pairs)."""
    from sparsepr_amd.kernels.n8_extension import wan_qkv_norm_rope_layout

    b, l, h, d = shape
    rng = np.random.default_rng(b * 1000 + h * d)
    c = h * d
    q, k, v = (_model_values(rng, (b, l, c), dtype, s) for s in (3.0, 1.0, 1.0))
    qw, kw = (_model_values(rng, (c,), dtype, 0.1) + 1.0 for _ in range(2))
    qw, kw = (torch.from_numpy(w.astype(np.float32)).to(dtype).float().numpy() for w in (qw, kw))
    ang = rng.uniform(-4.0, 4.0, (l, d // 2))
    fr, fi = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    args = [to_dev(x, dev, dtype) for x in (q, k, v, qw, kw)] + [to_dev(fr, dev), to_dev(fi, dev)]
    qo, ko, vo = wan_qkv_norm_rope_layout(*args, heads=h, epsilon=1e-6)
    assert qo.shape == (b, h, l, d) and qo.dtype == dtype
    rq, rk, rv = oracle.wan_qkv_norm_rope_layout(q, k, v, qw, kw, fr, fi, h, 1e-6, dtype=NAME[dtype])
    for got, ref in ((qo, rq), (ko, rk)):
        pr = ref.reshape(b, h, l, d // 2, 2)
        mag = np.repeat(np.hypot(pr[..., 0], pr[..., 1]), 2, axis=-1).reshape(ref.shape)
        _check(got, ref, mag, dtype, 0.9 if dtype != torch.float32 else 0.0)
    assert np.array_equal(vo.float().cpu().numpy(), rv)


_COSMOS_CASES = [(torch.bfloat16, (2, 257, 6, 128)), (torch.float16, (2, 257, 6, 128)),
                 (torch.float32, (2, 257, 6, 128)), (torch.bfloat16, (1, 100, 5, 64)),
                 (torch.bfloat16, (1, 64, 3, 256)), (torch.bfloat16, (1, 90, 4, 80))]


@pytest.mark.parametrize("dtype,shape", _COSMOS_CASES)
def test_cosmos25_qkv_norm_rope_bshd(dev, oracle, dtype, shape):
    """Lane-group paths for D = 64, 128, 256 (heads not a multiple of the heads per pass)
    in bf16, fp16 and fp32, and the per-row path (D = 80)."""
    from sparsepr_amd.kernels.n8_extension import cosmos25_qkv_norm_rope_bshd

    b, s, h, d = shape
    rng = np.random.default_rng(s * d + h)
    c = h * d
    q, k, v = (_model_values(rng, (b, s, c), dtype, sc) for sc in (2.0, 1.0, 1.0))
    qw = rng.uniform(0.8, 1.2, d).astype(np.float32)
    kw = rng.uniform(0.8, 1.2, d).astype(np.float32)
    freqs = rng.uniform(-20.0, 20.0, (s, d // 2))
    ang = np.concatenate((freqs, freqs), -1).reshape(s, 1, 1, d).astype(np.float32)
    qo, ko, vo = cosmos25_qkv_norm_rope_bshd(*[to_dev(x, dev, dtype) for x in (q, k, v)], to_dev(qw, dev),
                                             to_dev(kw, dev), to_dev(ang, dev), heads=h, epsilon=1e-6)
    assert qo.shape == (b, s, h, d) and qo.dtype == dtype
    rq, rk, rv = oracle.cosmos25_qkv_norm_rope_bshd(q, k, v, qw, kw, ang, h, 1e-6, dtype=NAME[dtype])
    half = d // 2
    for got, ref in ((qo, rq), (ko, rk)):
        m = np.hypot(ref[..., :half], ref[..., half:])
        mag = np.concatenate((m, m), -1)
        _check(got, ref, mag, dtype, 0.9 if dtype != torch.float32 else 0.0)
    assert np.array_equal(vo.float().cpu().numpy(), rv)


def test_qkv_argument_errors(dev):
    """The reference's argument checks (n8_ops.cu:356-497) with its messages."""
    from sparsepr_amd.kernels.n8_extension import cosmos25_qkv_norm_rope_bshd, wan_qkv_norm_rope_layout

    x = torch.zeros((1, 4, 24), device=dev, dtype=torch.bfloat16)
    w = torch.ones(24, device=dev, dtype=torch.bfloat16)
    f = torch.ones((4, 4), device=dev)
    with pytest.raises(RuntimeError, match="channels must divide"):
        wan_qkv_norm_rope_layout(x, x, x, w, w, f, f, heads=5, epsilon=1e-6)
    with pytest.raises(RuntimeError, match="head_dim must be even"):
        wan_qkv_norm_rope_layout(x, x, x, w, w, f, f, heads=8, epsilon=1e-6)
    with pytest.raises(RuntimeError, match=r"shape \[L,D/2\]"):
        wan_qkv_norm_rope_layout(x, x, x, w, w, f[:3], f[:3], heads=3, epsilon=1e-6)
    with pytest.raises(RuntimeError, match="must match the QKV dtype"):
        wan_qkv_norm_rope_layout(x, x, x, w.float(), w, f, f, heads=3, epsilon=1e-6)
    ang = torch.zeros((4, 1, 1, 8), device=dev)
    wf = torch.ones(8, device=dev)
    with pytest.raises(RuntimeError, match="epsilon must be positive"):
        cosmos25_qkv_norm_rope_bshd(x, x, x, wf, wf, ang, heads=3, epsilon=0.0)
    with pytest.raises(RuntimeError, match=r"shape \[S,1,1,D\]"):
        cosmos25_qkv_norm_rope_bshd(x, x, x, wf, wf, ang[:, :, :, :4], heads=3, epsilon=1e-6)
    with pytest.raises(RuntimeError, match="head_dim elements"):
        cosmos25_qkv_norm_rope_bshd(x, x, x, wf[:4], wf, ang, heads=3, epsilon=1e-6)
