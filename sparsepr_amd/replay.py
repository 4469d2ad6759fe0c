"""Real-tensor replay of one routed sparse-attention call.

The interchange format is the reference's "wan22_n8_sparse_attention_replay_v1"
(src/sparsepr/adapters/wan22.py:343-449): one post-routing attention call of a chosen
(generation step, layer, CFG branch), for a subset of heads, saved with torch.save as a
dict of metadata and CPU tensors:

    format, random_tensors, model, generation_step, layer, cfg_branch, heads, total_heads,
    tokens, head_dim, q_clusters, k_clusters, flashinfer_timings,
    q_sorted, k_sorted, v_sorted          [B, h, N, D]  cluster-sorted Q, K, V
    selected_mask                          [B, h, Qc, Kc] bool kept cluster pairs
    q_sizes, k_sizes                       [B, h, Qc] / [B, h, Kc]
    flashinfer_output_sorted               [B, h, N, D]  the attention output of that call

A capture made by the reference's pipeline (FlashInfer output) or by this package
(this package's output) replays through `replay_n8_attention`, which runs the
block-sparse attention kernel on the captured inputs and measures it against the
captured output: the offline kernel gate.  Captures are read with
torch.load(weights_only=True), which executes nothing from the file.
"""

from __future__ import annotations

import os
from pathlib import Path
from typing import Any

import torch

FORMAT = "wan22_n8_sparse_attention_replay_v1"
DEFAULT_CAPTURE_HEADS = "7,16,17,22"
_TENSOR_KEYS = ("q_sorted", "k_sorted", "v_sorted", "selected_mask", "q_sizes", "k_sizes",
                "flashinfer_output_sorted")
_META_KEYS = ("format", "random_tensors", "model", "generation_step", "layer", "cfg_branch", "heads",
              "total_heads", "tokens", "head_dim", "q_clusters", "k_clusters", "flashinfer_timings")
_CAPTURED = False


def parse_capture_heads(raw: str, total_heads: int) -> list[int]:
    """"all" or a comma list of head indices, validated against total_heads (wan22.py:380-399)."""
    if raw.strip().lower() == "all":
        heads = list(range(total_heads))
    else:
        heads = sorted({int(tok.strip()) for tok in raw.split(",") if tok.strip()})
    if not heads or heads[0] < 0 or heads[-1] >= total_heads:
        raise RuntimeError(f"WAN_N8_ATTENTION_CAPTURE_HEADS must select valid attention heads in "
                           f"[0, {total_heads}); got {heads}.")
    return heads


def capture_n8_attention_replay(path, *, q_permuted: torch.Tensor, k_permuted: torch.Tensor,
                                v_permuted: torch.Tensor, dynamic_map: torch.Tensor, q_sizes: torch.Tensor,
                                k_sizes: torch.Tensor, output_permuted: torch.Tensor, heads: list[int],
                                flashinfer_timings: dict | None = None, model: str | None = None,
                                generation_step: int = -1, layer: int = -1, cfg_branch: int = -1,
                                random_tensors: bool = False) -> Path:
    """Write one attention call in the v1 format for the given heads; returns the path."""
    total_heads = int(q_permuted.shape[1])
    if not heads or min(heads) < 0 or max(heads) >= total_heads:
        raise RuntimeError(f"capture heads {heads} outside [0, {total_heads}).")
    idx = torch.tensor(sorted(set(int(h) for h in heads)), dtype=torch.long, device=q_permuted.device)

    def pick(t: torch.Tensor) -> torch.Tensor:
        return t.index_select(1, idx.to(t.device)).detach().cpu().contiguous()

    payload: dict[str, Any] = {
        "format": FORMAT,
        "random_tensors": bool(random_tensors),
        "model": model,
        "generation_step": int(generation_step),
        "layer": int(layer),
        "cfg_branch": int(cfg_branch),
        "heads": [int(h) for h in idx.tolist()],
        "total_heads": total_heads,
        "tokens": int(q_permuted.shape[2]),
        "head_dim": int(q_permuted.shape[3]),
        "q_clusters": int(q_sizes.shape[-1]),
        "k_clusters": int(k_sizes.shape[-1]),
        "flashinfer_timings": dict(flashinfer_timings or {}),
        "q_sorted": pick(q_permuted),
        "k_sorted": pick(k_permuted),
        "v_sorted": pick(v_permuted),
        "selected_mask": pick(dynamic_map),
        "q_sizes": pick(q_sizes),
        "k_sizes": pick(k_sizes),
        "flashinfer_output_sorted": pick(output_permuted),
    }
    out = Path(path).expanduser()
    out.parent.mkdir(parents=True, exist_ok=True)
    torch.save(payload, out)
    return out


def maybe_capture_n8_attention_replay(attn: Any, **tensors) -> Path | None:
    """The environment-driven capture hook of an adapter (wan22.py:343-449): when
    WAN_N8_ATTENTION_REPLAY_CAPTURE names a path and this process has not captured yet,
    capture the call whose (step, layer, CFG branch) — read from attn's _svg_generation_step,
    _svg_layer_idx, _svg_cfg_branch — matches WAN_N8_ATTENTION_CAPTURE_STEP / _LAYER /
    _BRANCH (each defaulting to the call's own), for the heads in
    WAN_N8_ATTENTION_CAPTURE_HEADS (default 7,16,17,22).  tensors: the keyword arguments of
    capture_n8_attention_replay except heads and the metadata."""
    global _CAPTURED
    raw_path = os.environ.get("WAN_N8_ATTENTION_REPLAY_CAPTURE", "").strip()
    if not raw_path or _CAPTURED:
        return None
    step = int(getattr(attn, "_svg_generation_step", -1))
    layer = int(getattr(attn, "_svg_layer_idx", -1))
    branch = int(getattr(attn, "_svg_cfg_branch", -1))
    wanted = (int(os.environ.get("WAN_N8_ATTENTION_CAPTURE_STEP", str(step))),
              int(os.environ.get("WAN_N8_ATTENTION_CAPTURE_LAYER", str(layer))),
              int(os.environ.get("WAN_N8_ATTENTION_CAPTURE_BRANCH", str(branch))))
    if (step, layer, branch) != wanted:
        return None
    heads = parse_capture_heads(os.environ.get("WAN_N8_ATTENTION_CAPTURE_HEADS", DEFAULT_CAPTURE_HEADS),
                                int(tensors["q_permuted"].shape[1]))
    path = capture_n8_attention_replay(raw_path, heads=heads, model=getattr(attn, "_svg_model_name", None),
                                       generation_step=step, layer=layer, cfg_branch=branch, **tensors)
    _CAPTURED = True
    print(f"[WAN-N8-ATTENTION-CAPTURE] wrote {path} heads={heads} step={step} layer={layer} cfg={branch}",
          flush=True)
    return path


def reset_capture_state() -> None:
    """Allow another capture in this process (the hook captures once)."""
    global _CAPTURED
    _CAPTURED = False


def load_n8_attention_replay(path) -> dict:
    """Read a v1 capture (weights_only: nothing in the file is executed) and check that it is
    complete and self-consistent; raises ValueError naming the first problem."""
    payload = torch.load(Path(path).expanduser(), map_location="cpu", weights_only=True)
    if not isinstance(payload, dict) or payload.get("format") != FORMAT:
        found = payload.get("format") if isinstance(payload, dict) else type(payload).__name__
        raise ValueError(f"not a {FORMAT} capture (format={found!r}).")
    missing = [k for k in _META_KEYS + _TENSOR_KEYS if k not in payload]
    if missing:
        raise ValueError(f"capture is missing {missing}.")
    q, k, v = payload["q_sorted"], payload["k_sorted"], payload["v_sorted"]
    b, h, n, d = q.shape
    if k.shape != q.shape or v.shape != q.shape or payload["flashinfer_output_sorted"].shape != q.shape:
        raise ValueError(f"Q/K/V/output shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)} "
                         f"{tuple(payload['flashinfer_output_sorted'].shape)}.")
    qc, kc = int(payload["q_clusters"]), int(payload["k_clusters"])
    checks = {
        "selected_mask": (tuple(payload["selected_mask"].shape), (b, h, qc, kc)),
        "q_sizes": (tuple(payload["q_sizes"].shape), (b, h, qc)),
        "k_sizes": (tuple(payload["k_sizes"].shape), (b, h, kc)),
        "heads": (len(payload["heads"]), h),
        "tokens": (int(payload["tokens"]), n),
        "head_dim": (int(payload["head_dim"]), d),
    }
    for name, (got, want) in checks.items():
        if got != want:
            raise ValueError(f"capture field {name} is {got}, expected {want}.")
    for name, sizes in (("q_sizes", payload["q_sizes"]), ("k_sizes", payload["k_sizes"])):
        if bool((sizes < 0).any()) or bool((sizes.sum(-1) > n).any()):
            raise ValueError(f"capture {name} do not fit {n} tokens.")
    return payload


def replay_n8_attention(capture, *, device: str | torch.device = "cuda") -> dict:
    """Run the block-sparse attention on a capture's inputs and compare with its recorded
    output.  capture: a path or a loaded payload.  Returns the errors (max_abs, mean_abs,
    rel_l2 over all elements, min_cosine over rows) and the output [B, h, N, D]."""
    from .kmeans_utils import dynamic_block_sparse_fwd_flashinfer

    payload = capture if isinstance(capture, dict) else load_n8_attention_replay(capture)
    dev = torch.device(device)
    q, k, v = (payload[key].to(dev, torch.bfloat16).contiguous() for key in ("q_sorted", "k_sorted", "v_sorted"))
    out = dynamic_block_sparse_fwd_flashinfer(q, k, v, payload["selected_mask"].to(dev, torch.bool),
                                              payload["q_sizes"].to(dev), payload["k_sizes"].to(dev), is_cpu=False)
    ref = payload["flashinfer_output_sorted"].to(dev, torch.float32)
    got = out.float()
    diff = (got - ref).abs()
    cos = torch.nn.functional.cosine_similarity(got.flatten(0, 2), ref.flatten(0, 2), dim=-1, eps=1e-30)
    live = ref.flatten(0, 2).abs().amax(-1) > 0
    return {
        "max_abs": float(diff.max()),
        "mean_abs": float(diff.mean()),
        "rel_l2": float(torch.linalg.vector_norm(got - ref) / torch.linalg.vector_norm(ref).clamp_min(1e-30)),
        "min_cosine": float(cos[live].min()) if bool(live.any()) else 1.0,
        "output": out,
    }
