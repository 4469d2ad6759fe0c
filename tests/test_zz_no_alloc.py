"""The allocation-free block-sparse attention entry point against the workspace one,
through the C ABI: the same kernels on the same plan, so outputs and LSE must be
bit-identical.  Two calls in a row, the second smaller (the fixed plan array keeps
the first call's plan, which the second must fully replace), and an oversized
request refused before any launch."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _sizes(rng, n, total):
    w = rng.random(n) + 0.05
    w[::5] = 0.0  # empty clusters
    s = np.floor(w / w.sum() * total).astype(np.int64)
    s[np.argmax(w)] += total - s.sum()
    return s


def _case(dev, rng, bh_q, bh_kv, s, d, qn, kn):
    q = torch.randn((bh_q, s, d), device=dev).to(torch.bfloat16)
    k = torch.randn((bh_kv, s, d), device=dev).to(torch.bfloat16)
    v = torch.randn((bh_kv, s, d), device=dev).to(torch.bfloat16)
    qs = torch.from_numpy(np.stack([_sizes(rng, qn, s) for _ in range(bh_kv)])).to(dev, torch.int32)
    ks = torch.from_numpy(np.stack([_sizes(rng, kn, s) for _ in range(bh_kv)])).to(dev, torch.int32)
    m = torch.from_numpy(rng.random((bh_kv, qn, kn)) < 0.3).to(dev, torch.uint8)
    m[:, 0, 0] = 1
    return q, k, v, m, qs, ks


def _run(lib, fn, args, dev, ws=None):
    from sparsepr_amd import _lib

    q, k, v, m, qs, ks, bh_q, bh_kv, s, d, qn, kn = args
    out = torch.full_like(q, 3.0)
    lse = torch.full((bh_q, s), 5.0, device=dev)
    common = [q.data_ptr(), k.data_ptr(), v.data_ptr(), m.data_ptr(), qs.data_ptr(), ks.data_ptr(), bh_q, bh_kv, s,
              d, qn, kn, float(d) ** -0.5, None, None, out.data_ptr(), lse.data_ptr()]
    if ws is None:
        st = fn(*common, _lib.stream(dev))
    else:
        st = fn(*common, ws.data_ptr(), ws.numel(), _lib.stream(dev))
    assert st == 0, lib.spr_last_error()
    return out, lse


def test_noalloc_matches_workspace_entry_point_twice(dev):
    from sparsepr_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(5)
    for bh_q, bh_kv, s, d, qn, kn in [(8, 4, 3000, 128, 24, 96), (2, 2, 700, 128, 6, 11)]:
        print(f"noalloc case bh_q={bh_q} bh_kv={bh_kv} s={s} d={d} qn={qn} kn={kn}", flush=True)
        q, k, v, m, qs, ks = _case(dev, rng, bh_q, bh_kv, s, d, qn, kn)
        args = (q, k, v, m, qs, ks, bh_q, bh_kv, s, d, qn, kn)
        ws = torch.empty(int(lib.spr_block_sparse_attention_workspace(bh_kv, qn, kn)), dtype=torch.uint8, device=dev)
        ref_out, ref_lse = _run(lib, lib.spr_block_sparse_attention, args, dev, ws)
        out, lse = _run(lib, lib.spr_block_sparse_attention_noalloc, args, dev)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
        assert torch.equal(lse, ref_lse)
        assert not bool((out == 3.0).all(dim=-1).any())  # every row written


def test_noalloc_refuses_a_plan_beyond_the_fixed_array(dev):
    from sparsepr_amd import _lib

    lib = _lib.load()
    need = int(lib.spr_block_sparse_attention_workspace(64, 4096, 16384))
    assert need > (64 << 20)
    q = torch.zeros((64, 128, 128), dtype=torch.bfloat16, device=dev)
    st = lib.spr_block_sparse_attention_noalloc(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(),
                                                q.data_ptr(), q.data_ptr(), 64, 64, 128, 128, 4096, 16384, 0.1,
                                                None, None, q.data_ptr(), None, _lib.stream(dev))
    assert st == 3 and b"fixed plan array" in lib.spr_last_error()
