"""Block-graph execution of the Wan DiT with a selectable attention backend.

Mirrors models/fast_dit.py (the reference's fast path) at TP=1 with CFG as
batch 2, on one GPU:

  FAST_ATTN_IMPL   read once at import (models/fast_dit.py:43):
                     "hip"  (default) the gfx950 kernels of this package: QK-RMSNorm and
                            3D-RoPE fused into the flash self-attention, Q-RMSNorm fused
                            into the masked cross-attention (ops.self_attn_fused,
                            ops.cross_attn_fused)
                     "sdpa" torch's F.scaled_dot_product_attention after separate
                            QK-RMSNorm / RoPE ops (_sdpa, models/fast_dit.py:186-189)
  FAST_CROSS_IMPL  cross-attention backend, defaults to FAST_ATTN_IMPL (:45, :299-304)
  FAST_POINTWISE_IMPL  the block's pointwise chain (LayerNorms, _modulate, _gate, residual adds):
                     "hip"  (default) one fused pass per stage (ops.adaln) and the FFN's
                            tanh-GELU as the epilogue of its first GEMM
                     "eager" the separate torch ops of models/fast_dit.py:280-311

  _tp_rms_qk, _tp_rms  models/fast_dit.py:134-160 (TP=1: the all-reduce is the identity)
  _rope                models/fast_dit.py:163-169
  _modulate, _gate     models/fast_dit.py:172-181
  _FastBlock           models/fast_dit.py:260-311
  _FastCrossKV         models/fast_dit.py:464-477
  _FastHead, _FastPatch, FastWanDiT   models/fast_dit.py:480-697

Differences from the reference, all on purpose: no torch.compile (the
reference compiles each block for Neuron; here the hot ops are hand-written
kernels and the rest is eager PyTorch / hipBLASLt), the q/k/v projections of
the "hip" path run as one GEMM on concatenated weights (the kernels read q, k, v
as strided views of its output), cross-attention takes optional per-sample
text lengths, and the patch embedding (a Conv3d whose stride equals its
kernel) runs as the equivalent GEMM over gathered patches.
"""
import os
from typing import Optional, Sequence

import torch
import torch.nn.functional as F

from . import ops
from . import rope as _rope_mod
from .model import WanModel, sinusoidal_embedding_1d

FAST_ATTN_IMPL = os.environ.get("FAST_ATTN_IMPL", "hip")
FAST_CROSS_IMPL = os.environ.get("FAST_CROSS_IMPL", FAST_ATTN_IMPL)
FAST_POINTWISE_IMPL = os.environ.get("FAST_POINTWISE_IMPL", "hip")
IMPLS = ("hip", "sdpa")
for _name, _val in (("FAST_ATTN_IMPL", FAST_ATTN_IMPL), ("FAST_CROSS_IMPL", FAST_CROSS_IMPL)):
    if _val not in IMPLS:
        raise ValueError(f"{_name}={_val!r}: expected one of {IMPLS}")
if FAST_POINTWISE_IMPL not in ("hip", "eager"):
    raise ValueError(f"FAST_POINTWISE_IMPL={FAST_POINTWISE_IMPL!r}: expected 'hip' or 'eager'")


def _lin(x, layer):
    return F.linear(x, layer.weight, layer.bias)


def _tp_rms_qk(q, k, norm_q, norm_k):
    """q [B, Lq, C], k [B, Lk, C]: RMS over all C channels, fp32 stats, bf16 roundings."""
    qf, kf = q.float(), k.float()
    C = q.shape[-1]
    q_inv = torch.rsqrt(qf.pow(2).sum(-1, keepdim=True) / C + norm_q.eps)
    k_inv = torch.rsqrt(kf.pow(2).sum(-1, keepdim=True) / C + norm_k.eps)
    return (qf * q_inv).type_as(q) * norm_q.weight, (kf * k_inv).type_as(k) * norm_k.weight


def _tp_rms(x, norm):
    xf = x.float()
    ss = xf.pow(2).sum(-1, keepdim=True)
    return (xf * torch.rsqrt(ss / x.shape[-1] + norm.eps)).type_as(x) * norm.weight


def _rope(x, cos, sin):
    """x [B, L, n, d]; cos/sin [L, d/2] fp32: interleaved-pair rotation in fp32."""
    B, L, n, d = x.shape
    c = cos.view(1, L, 1, d // 2)
    s = sin.view(1, L, 1, d // 2)
    xp = x.float().reshape(B, L, n, d // 2, 2)
    xr, xi = xp[..., 0], xp[..., 1]
    out = torch.stack([xr * c - xi * s, xr * s + xi * c], dim=-1)
    return out.reshape(B, L, n, d).to(x.dtype)


def _modulate(x, shift, scale, num_frames):
    """x [B, L, C]; shift/scale [1, F, C] broadcast over each frame's tokens."""
    B, L, C = x.shape
    xv = x.view(B, num_frames, L // num_frames, C)
    return (xv * (1 + scale.unsqueeze(2)) + shift.unsqueeze(2)).view(B, L, C)


def _gate(y, gate, num_frames):
    B, L, C = y.shape
    return (y.view(B, num_frames, L // num_frames, C) * gate.unsqueeze(2)).view(B, L, C)


# ─── attention backends: q [B, Lq, n, d], k/v [B, Lk, n, d] -> [B, Lq, n, d] ───

def _sdpa(q, k, v, seqlen_k: Optional[Sequence[int]] = None, scale: Optional[float] = None):
    """torch SDPA over [B, L, n, d] views.  On a HIP device it runs in fp32 on contiguous
    [B, n, L, d] copies (torch's bf16 batched products over transposed views are not used)."""
    def one(qb, kb, vb):
        qt, kt, vt = (t.transpose(1, 2) for t in (qb, kb, vb))
        if qt.device.type == "cuda":
            qt, kt, vt = (t.float().contiguous() for t in (qt, kt, vt))
        return F.scaled_dot_product_attention(qt, kt, vt, scale=scale).transpose(1, 2).to(q.dtype)
    if seqlen_k is None:
        return one(q, k, v)
    return torch.cat([one(q[b:b + 1], k[b:b + 1, :n], v[b:b + 1, :n]) for b, n in enumerate(seqlen_k)], 0)


def _hip_self(q, k, v):
    return ops.flash_self_attn(q, k, v, q.shape[-1] ** -0.5, 0)


def _hip_cross(q, k, v, seqlen_k: Optional[torch.Tensor] = None):
    return ops.cross_attn(q, k, v, seqlen_k, q.shape[-1] ** -0.5)


def _hip_self_fused(q, k, v, norm_q, norm_k, cos, sin):
    return ops.self_attn_fused(q, k, v, norm_q.weight, norm_k.weight, norm_q.eps, cos, sin,
                               q.shape[-1] ** -0.5)


def _hip_cross_fused(q, k, v, norm_q, seqlen_k: Optional[torch.Tensor] = None):
    return ops.cross_attn_fused(q, k, v, norm_q.weight, norm_q.eps, seqlen_k, q.shape[-1] ** -0.5)


# ─── compiled-unit equivalents ────────────────────────────────────────────────

class _FastBlock:
    """One WanAttentionBlock forward (models/fast_dit.py:260-311) at TP=1."""

    def __init__(self, block, num_frames: int, attn_impl: str = FAST_ATTN_IMPL,
                 cross_impl: str = FAST_CROSS_IMPL, pointwise_impl: str = FAST_POINTWISE_IMPL):
        self.block = block
        self.num_frames = num_frames
        self.attn_impl = attn_impl
        self.cross_impl = cross_impl
        self.pointwise_impl = pointwise_impl
        sa = block.self_attn
        if attn_impl == "hip":
            self.w_qkv = torch.cat([sa.q.weight, sa.k.weight, sa.v.weight], 0).contiguous()
            self.b_qkv = torch.cat([sa.q.bias, sa.k.bias, sa.v.bias], 0).contiguous()

    def __call__(self, x, e0, cos, sin, ck, cv, seqlen_k=None):
        blk, nf = self.block, self.num_frames
        sa, ca = blk.self_attn, blk.cross_attn
        B, L, C = x.shape

        if self.pointwise_impl == "hip" and x.is_cuda:
            return self._fused(x, e0, cos, sin, ck, cv, seqlen_k)
        e = (blk.modulation.unsqueeze(0) + e0).chunk(6, dim=2)
        e = [t.squeeze(2) for t in e]  # each [1, F, C]

        # self-attention
        h = _modulate(blk.norm1(x).to(torch.bfloat16), e[0], e[1], nf)
        y = _lin(self._self_attn(h, cos, sin).reshape(B, L, C), sa.o)
        x = x + _gate(y, e[2], nf)

        # cross-attention; ck/cv [B, Lc, n, d] precomputed once per prompt (_FastCrossKV)
        h = blk.norm3(x)
        x = x + _lin(self._cross_attn(h, ck, cv, seqlen_k).reshape(B, L, C), ca.o)

        # FFN
        h = _modulate(blk.norm2(x).to(torch.bfloat16), e[3], e[4], nf)
        h = blk.ffn[1](_lin(h, blk.ffn[0]))
        y = _lin(h, blk.ffn[2])
        return x + _gate(y, e[5], nf)

    def _self_attn(self, h, cos, sin):
        blk = self.block
        sa = blk.self_attn
        B, L, C = h.shape
        n, d = sa.num_heads, sa.head_dim
        if self.attn_impl == "hip":
            qkv = F.linear(h, self.w_qkv, self.b_qkv)
            q, k, v = (qkv[..., i * C:(i + 1) * C].view(B, L, n, d) for i in range(3))
            return _hip_self_fused(q, k, v, sa.norm_q, sa.norm_k, cos, sin)
        q, k = _tp_rms_qk(_lin(h, sa.q), _lin(h, sa.k), sa.norm_q, sa.norm_k)
        v = _lin(h, sa.v).view(B, L, n, d)
        return _sdpa(_rope(q.view(B, L, n, d), cos, sin), _rope(k.view(B, L, n, d), cos, sin), v)

    def _cross_attn(self, h, ck, cv, seqlen_k):
        ca = self.block.cross_attn
        B, L, C = h.shape
        n, d = ca.num_heads, ca.head_dim
        if self.cross_impl == "hip":
            return _hip_cross_fused(_lin(h, ca.q).view(B, L, n, d), ck, cv, ca.norm_q, seqlen_k)
        q = _tp_rms(_lin(h, ca.q), ca.norm_q).view(B, L, n, d)
        return _sdpa(q, ck, cv, None if seqlen_k is None else seqlen_k.tolist())

    def _fused(self, x, e0, cos, sin, ck, cv, seqlen_k):
        """The same block with its pointwise chain in four fused adaLN passes
        (models/fast_dit.py:280, :294, :306-307, :311) and GELU in the FFN-up GEMM."""
        blk, nf = self.block, self.num_frames
        B, L, C = x.shape
        e = (blk.modulation.unsqueeze(0) + e0).reshape(nf, 6, C)      # rows 0..5 per frame
        x = x.contiguous()
        _, h = ops.adaln(x, e=e, frames=nf, shift_idx=0, scale_idx=1, eps=blk.norm1.eps)
        y = _lin(self._self_attn(h, cos, sin).reshape(B, L, C), blk.self_attn.o)
        x, h = ops.adaln(x, y, e, nf, gate_idx=2, ln_weight=blk.norm3.weight,
                         ln_bias=blk.norm3.bias, eps=blk.norm3.eps)
        y = _lin(self._cross_attn(h, ck, cv, seqlen_k).reshape(B, L, C), blk.cross_attn.o)
        x, h = ops.adaln(x, y, e, nf, shift_idx=3, scale_idx=4, eps=blk.norm2.eps)
        f0, f2 = blk.ffn[0], blk.ffn[2]
        h = torch._addmm_activation(f0.bias, h.view(B * L, C), f0.weight.t(), use_gelu=True)
        y = _lin(h.view(B, L, -1), f2)
        x, _ = ops.adaln(x, y, e, nf, gate_idx=5, norm=False)
        return x


class _FastCrossKV:
    """A block's cross-attention K (normalised) and V from the text context, once per prompt."""

    def __init__(self, block, cross_impl: str = FAST_CROSS_IMPL):
        self.block = block
        self.cross_impl = cross_impl

    def __call__(self, context):
        ca = self.block.cross_attn
        B, Lc, _ = context.shape
        n, d = ca.num_heads, ca.head_dim
        k = _lin(context, ca.k).view(B, Lc, n, d)
        if self.cross_impl == "hip":
            k = ops.rms_norm(k, ca.norm_k.weight, ca.norm_k.eps)
        else:
            k = _tp_rms(k.reshape(B, Lc, n * d), ca.norm_k).view(B, Lc, n, d)
        v = _lin(context, ca.v).view(B, Lc, n, d)
        return k, v


class _FastHead:
    """Head + unpatchify + CFG combine -> [C_out, F, H, W] (batch is [cond, uncond])."""

    def __init__(self, head, grid, patch_size, out_dim, guide_scale):
        self.head = head
        self.grid = grid
        self.patch_size = patch_size
        self.out_dim = out_dim
        self.guide_scale = guide_scale

    def __call__(self, x, e):
        hd = self.head
        f, h, w = self.grid
        p, q, r = self.patch_size
        c = self.out_dim
        m = (hd.modulation.unsqueeze(0) + e.unsqueeze(2)).chunk(2, dim=2)
        y = hd.head(_modulate(hd.norm(x), m[0].squeeze(2), m[1].squeeze(2), f))
        B = y.shape[0]
        y = y.view(B, f, h, w, p, q, r, c).permute(0, 7, 1, 4, 2, 5, 3, 6)
        y = y.reshape(B, c, f * p, h * q, w * r).to(torch.bfloat16)
        cond, uncond = y[0], y[1]
        return uncond + self.guide_scale * (cond - uncond)


class FastWanDiT:
    """Batched-CFG forward over a WanModel (models/fast_dit.py:561-697).

        fast = FastWanDiT(model, grid=(F, H/2, W/2), guide_scale=5.0)
        fast.set_context(ctx_cond, ctx_null)   # [1, 512, 4096] each, once per prompt
        noise_pred = fast(latent, t)           # latent [C, F, H, W], t scalar
    """

    def __init__(self, model: WanModel, grid, guide_scale: float, attn_impl: str = FAST_ATTN_IMPL,
                 cross_impl: str = FAST_CROSS_IMPL, pointwise_impl: str = FAST_POINTWISE_IMPL):
        self.model = model
        self.grid = tuple(int(g) for g in grid)
        self.num_frames = self.grid[0]
        self.seq_len = self.grid[0] * self.grid[1] * self.grid[2]
        dev = model.patch_embedding.weight.device
        self.device = dev
        head_dim = model.dim // model.num_heads
        self.cos, self.sin = _rope_mod.rope_tables(model.freqs, self.grid, head_dim, dev)
        self.blocks = [_FastBlock(b, self.num_frames, attn_impl, cross_impl, pointwise_impl)
                       for b in model.blocks]
        self.cross_kv = [_FastCrossKV(b, cross_impl) for b in model.blocks]
        self.head = _FastHead(model.head, self.grid, model.patch_size, model.out_dim, guide_scale)
        self.context = None
        self.seqlen_k = None

    def set_context(self, ctx_cond, ctx_null, context_lens: Optional[Sequence[int]] = None):
        """Text embedding and every block's cross K/V, once per prompt.  context_lens: the
        number of valid text tokens of (cond, uncond); None attends to all 512 tokens as the
        reference pipeline does."""
        ctx = torch.cat([ctx_cond, ctx_null], dim=0).to(self.device, torch.bfloat16)
        context = self.model.text_embedding(ctx)
        self.context = [kv(context) for kv in self.cross_kv]
        self.seqlen_k = None if context_lens is None else \
            torch.tensor(list(context_lens), dtype=torch.int32, device=self.device)

    def _time_embed(self, t):
        """Per-frame time embedding: frame 0 (the conditioning image) has t=0, the rest t."""
        m = self.model
        t_frames = torch.full((self.num_frames,), float(t), dtype=torch.float64)
        t_frames[0] = 0.0
        s = sinusoidal_embedding_1d(m.freq_dim, t_frames).to(torch.bfloat16).to(self.device).unsqueeze(0)
        e = m.time_embedding(s)                                # [1, F, C]
        e0 = m.time_projection(e).unflatten(2, (6, m.dim))     # [1, F, 6, C]
        return e, e0

    def patch(self, latent):
        """Patch embedding (a Conv3d with stride = kernel = patch_size) as one GEMM: gather
        each patch's in_dim x pt x ph x pw values in the weight's (c, t, h, w) order, then
        [L, in_dim*pt*ph*pw] x [dim, in_dim*pt*ph*pw]^T + bias.  Token order f, y, x."""
        conv = self.model.patch_embedding
        c, f, H, W = latent.shape
        pt, ph, pw = conv.kernel_size
        p = latent.to(torch.bfloat16).view(c, f // pt, pt, H // ph, ph, W // pw, pw)
        p = p.permute(1, 3, 5, 0, 2, 4, 6).reshape((f // pt) * (H // ph) * (W // pw), c * pt * ph * pw)
        x = F.linear(p, conv.weight.view(conv.weight.shape[0], -1), conv.bias)   # [L, C]
        return x.unsqueeze(0).expand(2, -1, -1).contiguous()

    def __call__(self, latent, t):
        assert self.context is not None, "call set_context() first"
        e, e0 = self._time_embed(t)
        x = self.patch(latent)
        for blk, (ck, cv) in zip(self.blocks, self.context):
            x = blk(x, e0, self.cos, self.sin, ck, cv, self.seqlen_k)
        return self.head(x, e)


def denoise(fast: FastWanDiT, latent: torch.Tensor, steps: int, shift: float,
            image_latent: Optional[torch.Tensor] = None, num_train_timesteps: int = 1000):
    """The TI2V denoising loop (inference_neuron_ti2v.py:450-531): UniPC over `steps`
    timesteps with the scheduler step on the device; if `image_latent` [C, 1, H, W] is
    given, frame 0 is reset to it after every step (the mask2 blend)."""
    from .unipc import FlowUniPC
    sched = FlowUniPC(num_train_timesteps=num_train_timesteps, shift=1.0)
    sched.set_timesteps(steps, shift=shift)
    if image_latent is not None:
        latent = latent.clone()
        latent[:, :1] = image_latent
    for t in sched.timesteps:
        noise_pred = fast(latent, t)
        latent = sched.step(noise_pred, latent)
        if image_latent is not None:
            latent[:, :1] = image_latent
    return latent
