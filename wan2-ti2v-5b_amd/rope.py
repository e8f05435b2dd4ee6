"""3D-RoPE angle tables of the Wan DiT (host side, built once per latent grid).

  rope_params   angle table p * theta^(-2j/dim), fp32    (wan/modules/rope_neuron.py:14-24)
  wan_freqs     frame / height / width tables, 44/42/42 (wan/modules/model.py:396-403)
  rope_tables   per-token cos/sin [L, 64] on the device (models/fast_dit.py:548-558)

The rotation itself runs on the GPU (ops.rope, or fused into the attention
kernels' Q/K load).  Tables are computed in fp32 on the host exactly as the
reference builds them and then copied to the device once.
"""
from typing import Sequence

import torch

THETA = 10000.0


def rope_params(max_seq_len: int, dim: int, theta: float = THETA) -> torch.Tensor:
    return torch.outer(torch.arange(max_seq_len).float(),
                       1.0 / torch.pow(theta, torch.arange(0, dim, 2).float().div(dim)))


def wan_freqs(head_dim: int = 128, max_seq_len: int = 1024) -> torch.Tensor:
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


def rope_tables(freqs: torch.Tensor, grid: Sequence[int], head_dim: int = 128,
                device="cpu"):
    """cos, sin as contiguous fp32 [L, head_dim/2] tensors on `device`, L = f*h*w.

    Token (t, y, x) of the latent grid has index t*h*w + y*w + x; its angles are
    [frame angles of t | height angles of y | width angles of x].
    """
    f, h, w = (int(g) for g in grid)
    c = head_dim // 2
    fr = freqs.detach().cpu().float().split([c - 2 * (c // 3), c // 3, c // 3], dim=1)
    if f > fr[0].shape[0] or h > fr[1].shape[0] or w > fr[2].shape[0]:
        raise ValueError(f"grid {grid} exceeds the angle table ({fr[0].shape[0]} positions)")
    ang = torch.cat([
        fr[0][:f].view(f, 1, 1, -1).expand(f, h, w, -1),
        fr[1][:h].view(1, h, 1, -1).expand(f, h, w, -1),
        fr[2][:w].view(1, 1, w, -1).expand(f, h, w, -1),
    ], dim=-1).reshape(f * h * w, c)
    return (torch.cos(ang).contiguous().to(device), torch.sin(ang).contiguous().to(device))
