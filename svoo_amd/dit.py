"""A random-init Wan2.1-shaped DiT in plain torch: the harness the SVOO processor runs in for one denoising step.

This is test and benchmark harness, not part of the accelerated path.  It reproduces the data flow the reference's
sparse Wan block drives (``svoo/models/wan/custom_models.py:23-109`` for the block, ``:112-195`` for the model) so
that the processor is called exactly as in a pipeline: ``block.attn1(hidden_states=..., rotary_emb=(cos, sin),
timestep=timestep)`` with ``rotary_emb`` shaped ``[1, S, 1, d]``.  The module names follow diffusers' Wan model
(``blocks[i].attn1.set_processor``, ``config.patch_size``), so :func:`svoo_amd.inference.replace_wan_attention`
installs processors into it as into a diffusers pipeline.  Weights are random (no checkpoint is available); the
shapes are Wan2.1-T2V-1.3B's by default.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class WanDiTConfig:
    """Wan2.1-T2V-1.3B transformer shape (diffusers ``WanTransformer3DModel`` config of that checkpoint)."""

    patch_size: Tuple[int, int, int] = (1, 2, 2)
    num_attention_heads: int = 12
    attention_head_dim: int = 128
    in_channels: int = 16
    out_channels: int = 16
    text_dim: int = 4096
    freq_dim: int = 256
    ffn_dim: int = 8960
    num_layers: int = 30
    eps: float = 1e-6
    rope_theta: float = 10000.0

    @property
    def dim(self) -> int:
        return self.num_attention_heads * self.attention_head_dim


class DenseWanAttnProcessor:
    """Dense attention processor with the Wan call signature (self- and cross-attention, no image branch)."""

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None,
                 timestep=None):
        ctx = hidden_states if encoder_hidden_states is None else encoder_hidden_states
        q = attn.norm_q(attn.to_q(hidden_states)).unflatten(2, (attn.heads, -1))
        k = attn.norm_k(attn.to_k(ctx)).unflatten(2, (attn.heads, -1))
        v = attn.to_v(ctx).unflatten(2, (attn.heads, -1))
        if rotary_emb is not None:
            q = apply_rope(q, *rotary_emb)
            k = apply_rope(k, *rotary_emb)
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           attn_mask=attention_mask)
        o = o.transpose(1, 2).flatten(2, 3).type_as(q)
        return attn.to_out[1](attn.to_out[0](o))


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation ``(x0, x1) -> (x0 c - x1 s, x0 s + x1 c)``; ``cos``/``sin`` repeat each angle twice."""
    x0, x1 = x.float().unflatten(-1, (-1, 2)).unbind(-1)
    c, s = cos[..., 0::2], sin[..., 0::2]
    return torch.stack((x0 * c - x1 * s, x0 * s + x1 * c), dim=-1).flatten(-2).type_as(x)


class FP32LayerNorm(nn.LayerNorm):
    """LayerNorm computed in float32 whatever the parameter dtype; returns the input's dtype."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = None if self.weight is None else self.weight.float()
        b = None if self.bias is None else self.bias.float()
        return F.layer_norm(x.float(), self.normalized_shape, w, b, self.eps).type_as(x)


class WanAttention(nn.Module):
    """Projections and norms of a Wan attention layer; the computation is delegated to its processor."""

    def __init__(self, dim: int, heads: int, eps: float):
        super().__init__()
        self.heads = heads
        self.to_q = nn.Linear(dim, dim)
        self.to_k = nn.Linear(dim, dim)
        self.to_v = nn.Linear(dim, dim)
        self.to_out = nn.ModuleList([nn.Linear(dim, dim), nn.Identity()])
        # qk_norm "rms_norm_across_heads": one RMSNorm over the full projection width
        self.norm_q = nn.RMSNorm(dim, eps=eps)
        self.norm_k = nn.RMSNorm(dim, eps=eps)
        self.add_k_proj = None
        self.add_v_proj = None
        self.processor = DenseWanAttnProcessor()

    def set_processor(self, processor) -> None:
        self.processor = processor

    def forward(self, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None,
                timestep=None):
        return self.processor(self, hidden_states, encoder_hidden_states, attention_mask, rotary_emb, timestep)


class WanBlock(nn.Module):
    """One Wan DiT block: modulated self-attention, cross-attention to the text, modulated FFN."""

    def __init__(self, cfg: WanDiTConfig):
        super().__init__()
        dim = cfg.dim
        self.norm1 = FP32LayerNorm(dim, eps=cfg.eps, elementwise_affine=False)
        self.attn1 = WanAttention(dim, cfg.num_attention_heads, cfg.eps)
        self.norm2 = FP32LayerNorm(dim, eps=cfg.eps, elementwise_affine=True)  # cross_attn_norm=True
        self.attn2 = WanAttention(dim, cfg.num_attention_heads, cfg.eps)
        self.norm3 = FP32LayerNorm(dim, eps=cfg.eps, elementwise_affine=False)
        self.ffn = nn.Sequential(nn.Linear(dim, cfg.ffn_dim), nn.GELU(approximate="tanh"), nn.Linear(cfg.ffn_dim, dim))
        self.scale_shift_table = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def forward(self, hidden_states, encoder_hidden_states, temb, rotary_emb, timestep=None):
        # custom_models.py:23-109 (the plain-torch branch): fp32 norms and modulation, bf16 activations
        mod = (self.scale_shift_table.float() + temb.float()).chunk(6, dim=1)
        shift, scale, gate, c_shift, c_scale, c_gate = mod
        dtype = hidden_states.dtype
        x = (self.norm1(hidden_states.float()) * (1 + scale) + shift).to(dtype)
        a = self.attn1(hidden_states=x, rotary_emb=rotary_emb, timestep=timestep)
        hidden_states = (hidden_states.float() + a.float() * gate).to(dtype)
        x = self.norm2(hidden_states.float()).to(dtype)
        hidden_states = hidden_states + self.attn2(hidden_states=x, encoder_hidden_states=encoder_hidden_states)
        x = (self.norm3(hidden_states.float()) * (1 + c_scale) + c_shift).to(dtype)
        f = self.ffn(x)
        return (hidden_states.float() + f.float() * c_gate).to(dtype)


def timestep_embedding(t: torch.Tensor, dim: int) -> torch.Tensor:
    """Sinusoidal embedding ``[cos(t w_i), sin(t w_i)]`` with ``w_i = 10000^(-i/(dim/2))``."""
    half = dim // 2
    w = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device, dtype=torch.float32) / half)
    a = t.float()[:, None] * w[None]
    return torch.cat([a.cos(), a.sin()], dim=-1)


def rope_tables(cfg: WanDiTConfig, frames: int, height: int, width: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """3-D RoPE of Wan: the head dim splits into (t, h, w) = (d - 4(d//6), 2(d//6), 2(d//6)) channels, each axis
    rotating its pairs by ``pos · theta^(-2i/axis_dim)``.  Returns ``cos, sin`` shaped ``[1, S, 1, d]`` with each
    angle repeated for the two elements of its pair."""
    d = cfg.attention_head_dim
    hw = 2 * (d // 6)
    dims = (d - 2 * hw, hw, hw)
    parts = []
    for n, ad in zip((frames, height, width), dims):
        inv = cfg.rope_theta ** (-torch.arange(0, ad, 2, dtype=torch.float64) / ad)
        parts.append(torch.arange(n, dtype=torch.float64)[:, None] * inv[None])  # [n, ad/2]
    t, h, w = parts
    ang = torch.cat([
        t[:, None, None, :].expand(frames, height, width, -1),
        h[None, :, None, :].expand(frames, height, width, -1),
        w[None, None, :, :].expand(frames, height, width, -1),
    ], dim=-1).reshape(frames * height * width, d // 2)
    ang = ang.repeat_interleave(2, dim=-1)
    return ang.cos().float().to(device)[None, :, None], ang.sin().float().to(device)[None, :, None]


class WanDiT(nn.Module):
    """Patch embedding, condition embedders, ``num_layers`` blocks, output head (``custom_models.py:112-195``)."""

    def __init__(self, cfg: WanDiTConfig = WanDiTConfig()):
        super().__init__()
        self.config = cfg
        dim = cfg.dim
        self.patch_embedding = nn.Conv3d(cfg.in_channels, dim, kernel_size=cfg.patch_size, stride=cfg.patch_size)
        self.time_embedder = nn.Sequential(nn.Linear(cfg.freq_dim, dim), nn.SiLU(), nn.Linear(dim, dim))
        self.time_proj = nn.Sequential(nn.SiLU(), nn.Linear(dim, 6 * dim))
        self.text_embedder = nn.Sequential(nn.Linear(cfg.text_dim, dim), nn.GELU(approximate="tanh"),
                                           nn.Linear(dim, dim))
        self.blocks = nn.ModuleList([WanBlock(cfg) for _ in range(cfg.num_layers)])
        self.norm_out = FP32LayerNorm(dim, eps=cfg.eps, elementwise_affine=False)
        self.scale_shift_table = nn.Parameter(torch.randn(1, 2, dim) / dim ** 0.5)
        self.proj_out = nn.Linear(dim, cfg.out_channels * math.prod(cfg.patch_size))
        self._rope = None

    def rope(self, f: int, h: int, w: int, device):
        key = (f, h, w, str(device))
        if self._rope is None or self._rope[0] != key:
            self._rope = (key, rope_tables(self.config, f, h, w, device))
        return self._rope[1]

    def forward(self, latents: torch.Tensor, timestep: torch.Tensor, text: torch.Tensor) -> torch.Tensor:
        b, _, f, h, w = latents.shape
        pt, ph, pw = self.config.patch_size
        f, h, w = f // pt, h // ph, w // pw
        rotary = self.rope(f, h, w, latents.device)
        x = self.patch_embedding(latents).flatten(2).transpose(1, 2).contiguous()
        temb = self.time_embedder(timestep_embedding(timestep, self.config.freq_dim).to(x.dtype))
        tproj = self.time_proj(temb).unflatten(1, (6, -1))
        ctx = self.text_embedder(text)
        for block in self.blocks:
            x = block(x, ctx, tproj, rotary, timestep=timestep)
        shift, scale = (self.scale_shift_table.float() + temb.float()[:, None]).chunk(2, dim=1)
        x = (self.norm_out(x.float()) * (1 + scale) + shift).to(x.dtype)
        x = self.proj_out(x)
        x = x.reshape(b, f, h, w, pt, ph, pw, -1).permute(0, 7, 1, 4, 2, 5, 3, 6)
        return x.flatten(6, 7).flatten(4, 5).flatten(2, 3)


def make_pipe(cfg: WanDiTConfig = WanDiTConfig(), device="cpu", dtype=torch.bfloat16, seed: int = 5,
              vae_scale_factor_temporal: int = 4, vae_scale_factor_spatial: int = 8):
    """A pipeline-shaped holder (``pipe.transformer``, VAE scale factors) around a random-init :class:`WanDiT`.

    Weights are drawn on ``device`` from ``torch.manual_seed(seed)``: normal(0, 0.02) for linear and conv weights,
    zero biases, unit norm weights."""
    torch.manual_seed(seed)
    with torch.device(device):
        model = WanDiT(cfg)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Conv3d)):
                m.weight.normal_(0.0, 0.02)
                if m.bias is not None:
                    m.bias.zero_()
    model = model.to(dtype).eval()
    return SimpleNamespace(transformer=model, transformer_2=None,
                           vae_scale_factor_temporal=vae_scale_factor_temporal,
                           vae_scale_factor_spatial=vae_scale_factor_spatial)


def latent_shape(cfg: WanDiTConfig, height: int, width: int, num_frames: int, vae_t: int = 4, vae_s: int = 8):
    """``[1, C, F, H, W]`` latent of a ``num_frames x height x width`` video (``F = 1 + (num_frames-1)//vae_t``)."""
    return (1, cfg.in_channels, 1 + (num_frames - 1) // vae_t, height // vae_s, width // vae_s)
