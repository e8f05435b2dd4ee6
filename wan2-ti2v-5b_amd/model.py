"""Wan2.2-TI2V-5B DiT module tree (the callers either side of the attention path).

Parameter names and shapes follow WanModel (wan/modules/model.py:292-403,
wan/configs/wan_ti2v_5B.py:14-29), so a state dict of the reference model
loads into it; nothing here depends on diffusers.  Weights are bf16 and can be
random-initialised directly on the device (std 0.02) for synthetic runs.

  WanRMSNorm       wan/modules/model.py:70-86   (weight [dim], eps 1e-6)
  WanLayerNorm     wan/modules/model.py:89-99
  WanAttention     wan/modules/model.py:102-181 (q, k, v, o, norm_q, norm_k)
  WanAttentionBlock wan/modules/model.py:184-258
  Head             wan/modules/model.py:261-289
  sinusoidal_embedding_1d wan/modules/model.py:15-25

The forward passes live in fast_dit.py (the block-graph execution of
models/fast_dit.py); this module only holds parameters.
"""
import math
from dataclasses import dataclass
from typing import Tuple

import torch
import torch.nn as nn

from . import rope as _rope


@dataclass(frozen=True)
class WanConfig:
    """Hyper-parameters of Wan2.2-TI2V-5B (wan/configs/wan_ti2v_5B.py:14-36)."""
    patch_size: Tuple[int, int, int] = (1, 2, 2)
    text_len: int = 512
    in_dim: int = 48
    dim: int = 3072
    ffn_dim: int = 14336
    freq_dim: int = 256
    text_dim: int = 4096
    out_dim: int = 48
    num_heads: int = 24
    num_layers: int = 30
    eps: float = 1e-6
    sample_shift: float = 5.0
    sample_guide_scale: float = 5.0
    num_train_timesteps: int = 1000

    @property
    def head_dim(self) -> int:
        return self.dim // self.num_heads


def sinusoidal_embedding_1d(dim: int, position: torch.Tensor) -> torch.Tensor:
    """[cos(p * 10000^(-j/half)) | sin(...)] in float64 (wan/modules/model.py:15-25)."""
    assert dim % 2 == 0
    half = dim // 2
    position = position.type(torch.float64)
    sinusoid = torch.outer(position, torch.pow(10000, -torch.arange(half).to(position).div(half)))
    return torch.cat([torch.cos(sinusoid), torch.sin(sinusoid)], dim=1)


class WanRMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class WanLayerNorm(nn.LayerNorm):
    def __init__(self, dim: int, eps: float = 1e-6, elementwise_affine: bool = False):
        super().__init__(dim, elementwise_affine=elementwise_affine, eps=eps)


class WanAttention(nn.Module):
    """Parameters of WanSelfAttention / WanCrossAttention."""

    def __init__(self, dim: int, num_heads: int, eps: float = 1e-6):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.eps = eps
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.norm_q = WanRMSNorm(dim, eps)
        self.norm_k = WanRMSNorm(dim, eps)


class WanAttentionBlock(nn.Module):
    def __init__(self, dim: int, ffn_dim: int, num_heads: int, eps: float = 1e-6):
        super().__init__()
        self.dim = dim
        self.ffn_dim = ffn_dim
        self.num_heads = num_heads
        self.eps = eps
        self.norm1 = WanLayerNorm(dim, eps)
        self.self_attn = WanAttention(dim, num_heads, eps)
        self.norm3 = WanLayerNorm(dim, eps, elementwise_affine=True)  # cross_attn_norm=True
        self.cross_attn = WanAttention(dim, num_heads, eps)
        self.norm2 = WanLayerNorm(dim, eps)
        self.ffn = nn.Sequential(nn.Linear(dim, ffn_dim), nn.GELU(approximate="tanh"),
                                 nn.Linear(ffn_dim, dim))
        self.modulation = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)


class Head(nn.Module):
    def __init__(self, dim: int, out_dim: int, patch_size, eps: float = 1e-6):
        super().__init__()
        self.dim = dim
        self.out_dim = out_dim
        self.patch_size = patch_size
        self.norm = WanLayerNorm(dim, eps)
        self.head = nn.Linear(dim, math.prod(patch_size) * out_dim)
        self.modulation = nn.Parameter(torch.randn(1, 2, dim) / dim ** 0.5)


class WanModel(nn.Module):
    """Parameter tree of the Wan DiT backbone (wan/modules/model.py:292-403)."""

    def __init__(self, cfg: WanConfig = WanConfig(), num_layers: int = None):
        super().__init__()
        self.cfg = cfg
        self.patch_size = cfg.patch_size
        self.dim = cfg.dim
        self.num_heads = cfg.num_heads
        self.freq_dim = cfg.freq_dim
        self.out_dim = cfg.out_dim
        self.eps = cfg.eps
        n_layers = cfg.num_layers if num_layers is None else num_layers
        self.patch_embedding = nn.Conv3d(cfg.in_dim, cfg.dim, kernel_size=cfg.patch_size,
                                         stride=cfg.patch_size)
        self.text_embedding = nn.Sequential(nn.Linear(cfg.text_dim, cfg.dim),
                                            nn.GELU(approximate="tanh"), nn.Linear(cfg.dim, cfg.dim))
        self.time_embedding = nn.Sequential(nn.Linear(cfg.freq_dim, cfg.dim), nn.SiLU(),
                                            nn.Linear(cfg.dim, cfg.dim))
        self.time_projection = nn.Sequential(nn.SiLU(), nn.Linear(cfg.dim, cfg.dim * 6))
        self.blocks = nn.ModuleList([WanAttentionBlock(cfg.dim, cfg.ffn_dim, cfg.num_heads, cfg.eps)
                                     for _ in range(n_layers)])
        self.head = Head(cfg.dim, cfg.out_dim, cfg.patch_size, cfg.eps)
        self.freqs = _rope.wan_freqs(cfg.head_dim)


def random_model(cfg: WanConfig = WanConfig(), num_layers: int = None, device="cuda",
                 dtype=torch.bfloat16, std: float = 0.02, seed: int = 0) -> WanModel:
    """A WanModel with seeded N(0, std) weights (LayerNorm/RMSNorm weights 1 + N(0, std),
    biases N(0, std)), created on `device` in `dtype` without a host copy of the weights."""
    with torch.device("meta"):
        m = WanModel(cfg, num_layers)
    m = m.to_empty(device=device).to(dtype)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or \
                    name.endswith("norm3.weight"):
                p.copy_(1 + std * torch.randn(p.shape, generator=g, device=device, dtype=torch.float32))
            elif name.endswith("modulation"):
                p.copy_(torch.randn(p.shape, generator=g, device=device, dtype=torch.float32) / cfg.dim ** 0.5)
            else:
                p.copy_(std * torch.randn(p.shape, generator=g, device=device, dtype=torch.float32))
    m.freqs = _rope.wan_freqs(cfg.head_dim)
    return m.eval().requires_grad_(False)
