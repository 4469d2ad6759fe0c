"""The replay gate on the GPU: a capture of this package's own attention replays exactly;
a capture holding the float64 closed-form output replays within the attention bound."""

import numpy as np
import pytest
import torch

from tests._helpers import to_dev

pytestmark = pytest.mark.gpu


def test_replay_gate(dev, oracle, tmp_path):
    from sparsepr_amd import replay
    from sparsepr_amd.kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    rng = np.random.default_rng(21)
    b, h, n, d, qc, kc = 1, 4, 3000, 128, 6, 11
    q, k, v = (oracle.to_bf16(rng.standard_normal((b, h, n, d)).astype(np.float32)) for _ in range(3))
    qs = np.stack([[np.diff(np.sort(np.concatenate(([0, n], rng.choice(n, qc - 1, replace=False)))))
                    for _ in range(h)]])
    ks = np.stack([[np.diff(np.sort(np.concatenate(([0, n], rng.choice(n, kc - 1, replace=False)))))
                    for _ in range(h)]])
    m = rng.random((b, h, qc, kc)) < 0.4
    m[..., 0] = True
    qt, kt, vt = (to_dev(x, dev, torch.bfloat16) for x in (q, k, v))
    out = dynamic_block_sparse_fwd_flashinfer(qt, kt, vt, to_dev(m, dev), to_dev(qs, dev), to_dev(ks, dev),
                                              is_cpu=False)
    call = dict(q_permuted=qt, k_permuted=kt, v_permuted=vt, dynamic_map=to_dev(m, dev), q_sizes=to_dev(qs, dev),
                k_sizes=to_dev(ks, dev))
    path = replay.capture_n8_attention_replay(tmp_path / "own.pt", heads=[0, 2, 3], output_permuted=out, **call)
    res = replay.replay_n8_attention(path, device=dev)
    assert res["max_abs"] == 0.0 and res["min_cosine"] > 0.9999
    assert torch.equal(res["output"], out[:, [0, 2, 3]])
    ref, _ = oracle.block_sparse_attention_dense(q, k, v, m, qs, ks, return_lse=True)
    path = replay.capture_n8_attention_replay(tmp_path / "ref.pt", heads=[1, 3], random_tensors=True,
                                              output_permuted=torch.from_numpy(ref.astype(np.float32)).bfloat16(),
                                              **call)
    res = replay.replay_n8_attention(path, device=dev)
    assert res["max_abs"] <= 2e-2 and res["rel_l2"] <= 5e-3 and res["min_cosine"] > 0.999
