"""attention() dispatch of the eager Wan modules (wan/modules/attention.py:190-237).

The reference routes q/k/v [B, L, n, d] to its NKI kernels when the tensors are
on the Neuron device and to F.scaled_dot_product_attention otherwise.  Here the
selector is explicit: impl "hip" (default; USE_HIP_KERNELS=1) runs the gfx950
kernels and requires HIP tensors, raising otherwise (no silent host fallback);
impl "sdpa" (USE_HIP_KERNELS=0) runs torch SDPA.  Unlike the reference's SDPA
fallback, which ignores k_lens with a warning (:222-227), both honour k_lens.
Host-side k_lens are checked against [1, Lk] as the reference's kernel_assert states;
k_lens already on the device are not read back (no host wait): the kernels clamp them.
"""
import os
from typing import Optional

import torch

from . import ops

USE_HIP_KERNELS = os.environ.get("USE_HIP_KERNELS", "1") == "1"


def attention(q, k, v, q_lens=None, k_lens: Optional[torch.Tensor] = None, dropout_p=0.,
              softmax_scale=None, q_scale=None, causal=False, window_size=(-1, -1),
              deterministic=False, dtype=torch.bfloat16, fa_version=None, is_cross_attn=False):
    """q [B, Lq, n, d], k/v [B, Lk, n, d] -> [B, Lq, n, d] (dtype bf16)."""
    if causal or dropout_p or window_size != (-1, -1) or q_scale is not None or q_lens is not None:
        raise NotImplementedError("attention(): causal, dropout, windows, q_scale and q_lens are "
                                  "not used by the Wan DiT and not implemented")
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if USE_HIP_KERNELS:
        q, k, v = (t.to(dtype) for t in (q, k, v))
        if k_lens is not None:
            if isinstance(k_lens, torch.Tensor) and k_lens.device.type == "cuda":
                # lengths already on the device are passed as they are: reading them here
                # would make the host wait for the stream; the kernels clamp each length
                # to [0, Lk] and give zeros for a sample with no keys
                return ops.cross_attn(q, k, v, k_lens.to(torch.int32), scale)
            lens = torch.as_tensor(k_lens, dtype=torch.int32)
            if int(lens.min()) < 1 or int(lens.max()) > k.shape[1]:
                raise ValueError(f"k_lens must be in [1, {k.shape[1]}], got {lens.tolist()}")
            return ops.cross_attn(q, k, v, lens.to(q.device), scale)
        if is_cross_attn:
            return ops.cross_attn(q, k, v, None, scale)
        return ops.flash_self_attn(q, k, v, scale, 0)
    from .fast_dit import _sdpa
    lens = None if k_lens is None else [int(x) for x in torch.as_tensor(k_lens).tolist()]
    q, k, v = (t.to(dtype) for t in (q, k, v))
    return _sdpa(q, k, v, lens, scale)


flash_attention = attention
