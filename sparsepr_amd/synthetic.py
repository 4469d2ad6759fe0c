"""Seeded synthetic video-token Q/K/V for the benchmark configurations.

Tokens are laid out frame by frame.  Each head draws `components` mixture means
~N(0, amp^2 I); the means drift along the frame axis as a random walk with step
std `step_std` per frame (frame-correlated video content).  Each token picks a
component uniformly.  Key means are correlated with the query means of the same
component (correlation `qk_corr`), value means are independent.  Token = mean +
noise_std * N(0, I).  Everything is generated on the device from a seeded torch
generator and stored as bf16.

amp sets the spread of cluster-level attention logits (about amp^2 in units of
q.k/sqrt(D)) and qk_corr the extra logit of a key cluster of the query's own
component (about qk_corr * amp^2 * sqrt(D)); together they set how much of the
attention mass top-p has to keep.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class VideoShape:
    heads: int
    frames: int
    height: int
    width: int
    dim: int = 128
    components: int = 400

    @property
    def tokens(self) -> int:
        return self.frames * self.height * self.width


# BASELINE configurations (latent frames x patch grid)
HUNYUAN = VideoShape(heads=24, frames=33, height=45, width=80, dim=128, components=400)  # 118,800 tokens
WAN = VideoShape(heads=40, frames=21, height=30, width=52, dim=128, components=200)       # 32,760 tokens
COSMOS = VideoShape(heads=40, frames=24, height=44, width=80, dim=128, components=300)    # 84,480 tokens
CPU_SMALL = VideoShape(heads=2, frames=4, height=32, width=32, dim=64, components=16)     # 4,096 tokens


def frame_gmm_qkv(shape: VideoShape, *, seed: int = 0, amp: float = 0.3, step_std: float = 0.1,
                  noise_std: float = 0.3, qk_corr: float = 1.0, device="cuda", dtype=torch.bfloat16,
                  heads: int | None = None):
    """Returns q, k, v of shape [1, H, N, D] in `dtype` (H = `heads` or shape.heads)."""
    h = shape.heads if heads is None else heads
    n_frames, per_frame, d, c = shape.frames, shape.height * shape.width, shape.dim, shape.components
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    outs = []
    for which in range(3):  # Q means, independent part of K means, V means
        base = amp * torch.randn(h, 1, c, d, device=device, generator=g)
        steps = step_std * torch.randn(h, n_frames, c, d, device=device, generator=g)
        steps[:, 0] = 0.0
        outs.append(base + torch.cumsum(steps, dim=1))  # [H, F, C, D]
    q_means, k_free, v_means = outs
    k_means = qk_corr * q_means + (1.0 - qk_corr ** 2) ** 0.5 * k_free
    frame_of = torch.arange(n_frames, device=device).repeat_interleave(per_frame)  # [N]

    def draw(means):
        comp = torch.randint(0, c, (h, n_frames * per_frame), device=device, generator=g)
        idx = frame_of.unsqueeze(0) * c + comp  # flat index into [F*C]
        mu = torch.gather(means.reshape(h, n_frames * c, d), 1, idx.unsqueeze(-1).expand(-1, -1, d))
        return (mu + noise_std * torch.randn(h, n_frames * per_frame, d, device=device, generator=g)).to(dtype)

    q = draw(q_means)
    k = draw(k_means)
    v = draw(v_means)
    return q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)


def gmm_points(batch: int, n: int, dim: int, components: int, *, seed: int = 0, std: float = 0.25,
               device="cuda", dtype=torch.bfloat16):
    """per batch a `components`-component Gaussian mixture with
    means ~N(0, 1), std `std`, mixture weights ~ Dirichlet(1).  [B, N, D]."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    means = torch.randn(batch, components, dim, device=device, generator=g)
    expo = -torch.log(torch.rand(batch, components, device=device, generator=g).clamp_min(1e-12))
    weights = expo / expo.sum(-1, keepdim=True)  # Dirichlet(1) via normalised exponentials
    comp = torch.multinomial(weights, n, replacement=True, generator=g)
    mu = torch.gather(means, 1, comp.unsqueeze(-1).expand(-1, -1, dim))
    return (mu + std * torch.randn(batch, n, dim, device=device, generator=g)).to(dtype)


def first_k_indices(n: int, k: int, seed: int) -> torch.Tensor:
    """First k entries of a seeded permutation of range(n) (CPU generator)."""
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randperm(n, generator=g)[:k]
