"""The wan22_n8_sparse_attention_replay_v1 interchange (wan22.py:343-449): writing,
loading with weights_only, schema checks and the environment-driven capture hook.  CPU
tensors only; the GPU replay gate is in test_gpu_replay.py."""

import pytest
import torch

from sparsepr_amd import replay


def _call(b=1, h=4, n=64, d=16, qc=3, kc=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    qs = torch.tensor([[20, 30, 14]] * h).unsqueeze(0).expand(b, h, qc).contiguous()
    ks = torch.tensor([[10, 10, 20, 4, 20]] * h).unsqueeze(0).expand(b, h, kc).contiguous()
    return dict(q_permuted=torch.randn((b, h, n, d), generator=g).bfloat16(),
                k_permuted=torch.randn((b, h, n, d), generator=g).bfloat16(),
                v_permuted=torch.randn((b, h, n, d), generator=g).bfloat16(),
                dynamic_map=torch.rand((b, h, qc, kc), generator=g) < 0.5,
                q_sizes=qs, k_sizes=ks, output_permuted=torch.randn((b, h, n, d), generator=g).bfloat16())


def test_capture_round_trip(tmp_path):
    call = _call()
    path = replay.capture_n8_attention_replay(tmp_path / "a" / "cap.pt", heads=[3, 1], model="wan", layer=7,
                                              generation_step=2, cfg_branch=0, flashinfer_timings={"run_ms": 1.5},
                                              **call)
    p = replay.load_n8_attention_replay(path)
    assert p["format"] == replay.FORMAT and p["heads"] == [1, 3] and p["total_heads"] == 4
    assert (p["tokens"], p["head_dim"], p["q_clusters"], p["k_clusters"]) == (64, 16, 3, 5)
    assert p["layer"] == 7 and p["generation_step"] == 2 and p["flashinfer_timings"] == {"run_ms": 1.5}
    assert torch.equal(p["q_sorted"], call["q_permuted"][:, [1, 3]])
    assert torch.equal(p["selected_mask"], call["dynamic_map"][:, [1, 3]])
    assert torch.equal(p["flashinfer_output_sorted"], call["output_permuted"][:, [1, 3]])


def test_load_rejects_malformed(tmp_path):
    call = _call()
    path = replay.capture_n8_attention_replay(tmp_path / "cap.pt", heads=[0], **call)
    payload = torch.load(path, weights_only=True)
    for key, value, msg in (("format", "other_v2", "not a"), ("k_sizes", torch.ones((1, 1, 4), dtype=torch.long),
                                                               "k_sizes"),
                            ("q_sizes", torch.tensor([[[60, 30, 14]]]), "do not fit"),
                            ("tokens", 65, "tokens")):
        bad = dict(payload)
        bad[key] = value
        torch.save(bad, tmp_path / "bad.pt")
        with pytest.raises(ValueError, match=msg):
            replay.load_n8_attention_replay(tmp_path / "bad.pt")
    bad = dict(payload)
    del bad["v_sorted"]
    torch.save(bad, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="missing"):
        replay.load_n8_attention_replay(tmp_path / "bad.pt")


def test_capture_hook_environment(tmp_path, monkeypatch):
    class Attn:
        _svg_generation_step, _svg_layer_idx, _svg_cfg_branch, _svg_model_name = 3, 10, 1, "wan2.2"

    replay.reset_capture_state()
    call = _call(h=24)
    assert replay.maybe_capture_n8_attention_replay(Attn(), **call) is None  # no path: off
    monkeypatch.setenv("WAN_N8_ATTENTION_REPLAY_CAPTURE", str(tmp_path / "hook.pt"))
    monkeypatch.setenv("WAN_N8_ATTENTION_CAPTURE_LAYER", "11")
    assert replay.maybe_capture_n8_attention_replay(Attn(), **call) is None  # another layer
    monkeypatch.setenv("WAN_N8_ATTENTION_CAPTURE_LAYER", "10")
    path = replay.maybe_capture_n8_attention_replay(Attn(), **call)
    p = replay.load_n8_attention_replay(path)
    assert p["heads"] == [7, 16, 17, 22] and p["model"] == "wan2.2" and p["cfg_branch"] == 1
    assert replay.maybe_capture_n8_attention_replay(Attn(), **call) is None  # once per process
    replay.reset_capture_state()
    monkeypatch.setenv("WAN_N8_ATTENTION_CAPTURE_HEADS", "all")
    assert replay.load_n8_attention_replay(replay.maybe_capture_n8_attention_replay(Attn(), **call))["heads"] == \
        list(range(24))
    replay.reset_capture_state()


def test_parse_capture_heads():
    assert replay.parse_capture_heads(" 3, 1,3 ", 4) == [1, 3]
    for raw in ("", "4", "-1,2"):
        with pytest.raises(RuntimeError, match="valid attention heads"):
            replay.parse_capture_heads(raw, 4)
