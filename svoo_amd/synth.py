"""Seeded synthetic Q/K/V and sparsity profiles for the benchmark configurations.

Inputs are drawn on the CPU with ``torch.Generator`` in float32 (one generator per
head, so any subset of heads can be regenerated on its own) and then cast, so a
GPU run and a CPU baseline see identical data.

Per head ``h``: ``M`` component centres ``mu_Q, mu_K, mu_V ~ N(0, I_d)``; one
component ``z_n`` per token shared by Q, K and V (this is what gives the QK
co-cluster structure); ``x_n = mu_{z_n} + 0.3 * eps``; configurations with a
drift add ``f * delta_h`` with ``delta_h ~ N(0, 0.02^2 I)`` and frame index
``f = n // frame_size``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch


@dataclass(frozen=True)
class SynthConfig:
    name: str
    seed: int
    heads: int
    frames: int
    frame_h: int
    frame_w: int
    head_dim: int
    mixture: int
    num_q_centroids: int
    num_k_centroids: int
    kmeans_iters: int
    density_lo: float
    density_hi: float
    drift: bool
    dtype: str  # "bf16" or "fp32"
    text_tokens: int = 0
    warm_start: bool = False

    @property
    def frame_size(self) -> int:
        return self.frame_h * self.frame_w

    @property
    def video_tokens(self) -> int:
        return self.frames * self.frame_size

    @property
    def tokens(self) -> int:
        return self.video_tokens + self.text_tokens

    def dense_flops(self) -> float:
        """``4 * H * N^2 * d``: QK^T and PV of dense attention at this shape."""
        return 4.0 * self.heads * float(self.tokens) ** 2 * self.head_dim


CONFIGS = {
    "C1": SynthConfig("C1-cpu-plumbing", 1, 2, 3, 30, 52, 128, 32, 32, 64, 5, 0.25, 0.25, False, "fp32"),
    "C2": SynthConfig("C2-wan2.1-1.3B-480p", 2, 12, 21, 30, 52, 128, 256, 100, 500, 5, 0.05, 0.4, True, "bf16"),
    "C3": SynthConfig("C3-wan2.1-14B-720p", 3, 40, 21, 45, 80, 128, 256, 100, 1000, 5, 0.05, 0.3, True, "bf16",
                      warm_start=True),
    "C4": SynthConfig("C4-hunyuan-720p-129f", 4, 24, 33, 45, 80, 128, 256, 200, 1000, 5, 0.05, 0.3, True, "bf16",
                      text_tokens=256),
}


def _head_generator(seed: int, head: int, stream: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed * 1_000_003 + head * 97 + stream)
    return g


def make_head_qkv(cfg: SynthConfig, head: int, tokens: Optional[int] = None) -> Tuple[torch.Tensor, ...]:
    """float32 ``(q, k, v)`` of shape ``[N, d]`` for one head (CPU)."""
    n = cfg.tokens if tokens is None else tokens
    d = cfg.head_dim
    g = _head_generator(cfg.seed, head, 0)
    mus = [torch.randn(cfg.mixture, d, generator=g) for _ in range(3)]
    z = torch.randint(0, cfg.mixture, (n,), generator=g)
    out = []
    frame = (torch.arange(n) // cfg.frame_size).to(torch.float32)[:, None]
    for t in range(3):
        x = mus[t][z] + 0.3 * torch.randn(n, d, generator=g)
        if cfg.drift:
            delta = 0.02 * torch.randn(d, generator=g)
            x = x + frame * delta[None, :]
        out.append(x)
    return tuple(out)


def make_qkv(cfg: SynthConfig, heads: Optional[Sequence[int]] = None, device="cpu", tokens: Optional[int] = None):
    """``(q, k, v)`` of shape ``[1, len(heads), N, d]`` in the config dtype on ``device``."""
    heads = list(range(cfg.heads)) if heads is None else list(heads)
    dt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    n = cfg.tokens if tokens is None else tokens
    qkv = [torch.empty(1, len(heads), n, cfg.head_dim, dtype=dt, device=device) for _ in range(3)]
    for i, h in enumerate(heads):
        hq = make_head_qkv(cfg, h, tokens)
        for t in range(3):
            qkv[t][0, i].copy_(hq[t].to(dt))
    return tuple(qkv)


def make_qkv_device(cfg: SynthConfig, device, seed_offset: int = 0):
    """``(q, k, v)`` ``[1, H, N, d]`` in the config dtype, drawn on ``device`` with a seeded device generator.

    Same mixture as :func:`make_head_qkv`, all heads at once (the full-size benchmark shapes take
    seconds on the CPU).  The values differ from the CPU generator's; a CPU comparison copies
    heads of these tensors back to the host.
    """
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(cfg.seed * 1_000_003 + 7 + seed_offset)
    h, n, d, m = cfg.heads, cfg.tokens, cfg.head_dim, cfg.mixture
    dt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    z = torch.randint(0, m, (h, n), generator=g, device=dev)
    frame = (torch.arange(n, device=dev) // cfg.frame_size).to(torch.float32)[None, :, None]
    out = []
    for _ in range(3):
        mu = torch.randn(h, m, d, generator=g, device=dev)
        x = torch.gather(mu, 1, z[:, :, None].expand(h, n, d))
        x.add_(torch.randn(h, n, d, generator=g, device=dev), alpha=0.3)
        if cfg.drift:
            delta = 0.02 * torch.randn(h, 1, d, generator=g, device=dev)
            x.add_(frame * delta)
        out.append(x.to(dt)[None].contiguous())
        del x, mu
    return tuple(out)


def head_densities(cfg: SynthConfig, heads: Optional[Sequence[int]] = None) -> List[float]:
    """Per-head density ``rho_h ~ U[lo, hi]`` (seeded), used as the minimum key-cluster ratio."""
    g = torch.Generator(device="cpu")
    g.manual_seed(cfg.seed * 7919 + 13)
    rho = cfg.density_lo + (cfg.density_hi - cfg.density_lo) * torch.rand(cfg.heads, generator=g, dtype=torch.float64)
    heads = list(range(cfg.heads)) if heads is None else list(heads)
    return [float(rho[h]) for h in heads]


def init_indices(cfg: SynthConfig, bh: int, num_clusters: int, tokens: int, stream: int) -> torch.Tensor:
    """Seeded initial token indices ``[bh, num_clusters]`` (the reference draws them with ``torch.randint``)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(cfg.seed * 104729 + stream)
    return torch.randint(0, tokens, (bh, num_clusters), generator=g, dtype=torch.int64)


def perturb_centroids(cfg: SynthConfig, centroids: torch.Tensor, stream: int, scale: float = 0.05) -> torch.Tensor:
    """Warm start: ``C + N(0, (scale * rms(C))^2)`` per head, drawn on the CPU, returned on ``centroids.device``."""
    c = centroids.detach().to("cpu", torch.float32)
    g = torch.Generator(device="cpu")
    g.manual_seed(cfg.seed * 15485863 + stream)
    rms = c.pow(2).mean(dim=(-1, -2), keepdim=True).sqrt()
    noisy = c + scale * rms * torch.randn(c.shape, generator=g)
    return noisy.to(centroids.dtype).to(centroids.device)
