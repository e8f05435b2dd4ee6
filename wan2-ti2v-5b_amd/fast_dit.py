"""The Wan DiT forward around the attention path, on one GPU, with selectable backends.

This is the block-level drop-in for the reference's fast path (models/fast_dit.py) at
TP=1, with classifier-free guidance run as batch 2 ([cond, uncond]).  The backends are
chosen once at import, under the reference's selector names (models/fast_dit.py:43-45):

  FAST_ATTN_IMPL       "hip" (default): QK-RMSNorm, 3D-RoPE and the self-attention in the
                       gfx950 kernels (ops.self_attn_fused); "sdpa": torch ops with the
                       reference's rounding points and F.scaled_dot_product_attention
  FAST_CROSS_IMPL      the cross-attention backend (default: FAST_ATTN_IMPL); "hip" runs the
                       Q-RMSNorm + masked cross-attention kernel (ops.cross_attn_fused)
  FAST_POINTWISE_IMPL  "hip" (default): each pointwise stage of a block is one fused pass
                       (ops.adaln) and GELU is the FFN-up GEMM's epilogue; "eager": torch ops
  FAST_QKV_IMPL        with "hip" attention, the q/k/v projection: "hipblaslt" (default) or
                       "hip", the gfx950 GEMM that also emits the QK-RMSNorm sums of squares

A block (models/fast_dit.py:270-311) is organised here as four pointwise stages between
its GEMM groups, e the block's per-frame modulation rows:

  stage 1   h = LN1(x) * (1 + e1) + e0                 -> q/k/v, self-attention, O projection -> y
  stage 2   x = x + y * e2;  h = LN3(x)                -> cross q, cross-attention, O         -> y
  stage 3   x = x + y;       h = LN2(x) * (1 + e4) + e3 -> FFN up + GELU, FFN down           -> y
  stage 4   x = x + y * e5

Both pointwise implementations round to bf16 where the reference's eager graph does, and
both attention backends see the same q, k, v.  Not done as the reference does: no
torch.compile (the hot ops are hand-written kernels, the GEMMs hipBLASLt); with "hip" the
q/k/v projections are one GEMM on concatenated weights, read by the kernels as strided
views; cross-attention accepts per-sample text lengths; the patch embedding (a Conv3d with
stride equal to its kernel) is the equivalent GEMM over gathered patches.
"""
import math
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
# The fused q/k/v projection of the "hip" self-attention: "hipblaslt" (default), or "hip", the
# gfx950 GEMM whose epilogue emits the QK-RMSNorm sums of squares (ops.qkv_proj_sumsq), so the
# q statistics pass disappears; it measures 0.70 ms against hipBLASLt's 0.60 ms at the
# B=2, L=7854 shape, more than the 9-20 us the q read costs, hence not the default.
FAST_QKV_IMPL = os.environ.get("FAST_QKV_IMPL", "hipblaslt")
IMPLS = ("hip", "sdpa")
for _name, _val in (("FAST_ATTN_IMPL", FAST_ATTN_IMPL), ("FAST_CROSS_IMPL", FAST_CROSS_IMPL)):
    if _val not in IMPLS:
        raise ValueError(f"{_name}={_val!r}: expected one of {IMPLS}")
if FAST_POINTWISE_IMPL not in ("hip", "eager"):
    raise ValueError(f"FAST_POINTWISE_IMPL={FAST_POINTWISE_IMPL!r}: expected 'hip' or 'eager'")
if FAST_QKV_IMPL not in ("hipblaslt", "hip"):
    raise ValueError(f"FAST_QKV_IMPL={FAST_QKV_IMPL!r}: expected 'hipblaslt' or 'hip'")


def _linear(x, layer):
    return F.linear(x, layer.weight, layer.bias)


# ─── torch ops of the "sdpa" / "eager" side, rounding as the reference's graph ──────

def _rms_normalize(x, weight, eps):
    """RMS normalisation over the last axis (every head of a token): statistics in fp32, the
    normalised row rounded to x's dtype, then scaled by `weight` in that dtype (the
    reference's _tp_rms / _tp_rms_qk, models/fast_dit.py:134-160, whose all-reduce is the
    identity at TP=1)."""
    xf = x.float()
    mean_sq = torch.sum(xf * xf, dim=-1, keepdim=True) / x.shape[-1]
    return (xf * torch.rsqrt(mean_sq + eps)).to(x.dtype) * weight


def _rope(x, cos, sin):
    """3D-RoPE of x [B, L, H, D]: channel pair (2j, 2j+1) of token l is turned by the angle
    whose cosine and sine are cos[l, j], sin[l, j] (fp32 tables [L, D/2]); fp32 arithmetic,
    one rounding back to x's dtype (models/fast_dit.py:163-169)."""
    pairs = x.float().unflatten(-1, (-1, 2))
    re, im = pairs[..., 0], pairs[..., 1]
    c, s = cos[:, None, :], sin[:, None, :]          # broadcast over batch and heads
    return torch.stack((re * c - im * s, re * s + im * c), dim=-1).flatten(-2).to(x.dtype)


def _by_frame(t, num_frames):
    """[B, L, C] -> [B, F, L/F, C]: each latent frame's tokens are contiguous."""
    return t.unflatten(1, (num_frames, t.shape[1] // num_frames))


def _eager_stage(x, y, e, num_frames, gate=-1, shift=-1, scale=-1, ln=None, norm=True, mod=None):
    """One pointwise stage as separate torch ops (models/fast_dit.py:172-181,280,294,306-311);
    the same contract as ops.adaln.  e: [F, n, C] rows; returns (r, h):
        r = x, x + y, or x + y * e[gate]            (product and sum each rounded)
        h = ln(r), then h * (1 + m[scale]) + m[shift] per frame   (None when norm is False)
    with m = e, or `mod` [F, n', C] when the modulation belongs to the stage that follows
    (the next block's norm1, or the output head)."""
    m = e if mod is None else mod

    def row(t, i):
        return t[:, i].unsqueeze(1)                  # [F, 1, C] against [B, F, L/F, C]
    r = x
    if y is not None:
        if gate >= 0:
            y = (_by_frame(y, num_frames) * row(e, gate)).flatten(1, 2)
        r = x + y
    if not norm:
        return r, None
    h = ln(r)
    if shift >= 0:
        h = (_by_frame(h, num_frames) * (1 + row(m, scale)) + row(m, shift)).flatten(1, 2)
    return r, h


def _hip_stage(x, y, e, num_frames, gate=-1, shift=-1, scale=-1, ln=None, norm=True, mod=None):
    """The same stage as one fused pass over the residual stream (wan_adaln / wan_adaln_ex)."""
    w = b = None
    if ln is not None and ln.weight is not None:
        w, b = ln.weight, ln.bias
    eps = ln.eps if ln is not None else 1e-6
    return ops.adaln(x, y, e, num_frames, gate_idx=gate, shift_idx=shift, scale_idx=scale,
                     ln_weight=w, ln_bias=b, eps=eps, norm=norm, e_mod=mod)


def _ffn_eager(h, ffn):
    return _linear(ffn[1](_linear(h, ffn[0])), ffn[2])


def _ffn_gelu_epilogue(h, ffn):
    """FFN with the tanh-GELU applied in the first GEMM's epilogue (hipBLASLt)."""
    B, L, C = h.shape
    up = torch._addmm_activation(ffn[0].bias, h.reshape(B * L, C), ffn[0].weight.t(), use_gelu=True)
    return _linear(up.view(B, L, -1), ffn[2])


# ─── attention backends: q [B, Lq, n, d], k/v [B, Lk, n, d] -> [B, Lq, n, d] ───────

def _sdpa(q, k, v, seqlen_k: Optional[Sequence[int]] = None, scale: Optional[float] = None):
    """torch SDPA over [B, L, n, d] views (the reference's _sdpa, models/fast_dit.py:186-189).
    On a HIP device it runs in fp32 on contiguous [B, n, L, d] copies (torch's bf16 batched
    products over transposed views are not used).  seqlen_k: keys per sample."""
    def one(qb, kb, vb):
        qt, kt, vt = (t.transpose(1, 2) for t in (qb, kb, vb))
        if qt.device.type == "cuda":
            qt, kt, vt = (t.float().contiguous() for t in (qt, kt, vt))
        return F.scaled_dot_product_attention(qt, kt, vt, scale=scale).transpose(1, 2).to(q.dtype)
    if seqlen_k is None:
        return one(q, k, v)
    return torch.cat([one(q[b:b + 1], k[b:b + 1, :n], v[b:b + 1, :n]) for b, n in enumerate(seqlen_k)], 0)


def _pack_qkv(sa):
    """One [3C, C] weight and [3C] bias for the fused q/k/v projection.  The q, k and v
    parameters become views into them (same names, shapes and values, so state dicts still
    load), so the weights are held once rather than twice.  Packed once per module."""
    packed = getattr(sa, "_wan_qkv_packed", None)
    layers = (sa.q, sa.k, sa.v)
    if packed is not None and all(l.weight.data_ptr() == packed[0][i * l.weight.shape[0]:].data_ptr()
                                  for i, l in enumerate(layers)):
        return packed
    w = torch.cat([l.weight.detach() for l in layers], 0).contiguous()
    b = torch.cat([l.bias.detach() for l in layers], 0).contiguous()
    off = 0
    for l in layers:
        n = l.weight.shape[0]
        l.weight.data = w[off:off + n]
        l.bias.data = b[off:off + n]
        off += n
    sa._wan_qkv_packed = (w, b)
    return w, b


class _FastBlock:
    """One WanAttentionBlock forward (the reference's _FastBlock, models/fast_dit.py:260-311)
    at TP=1, as the four stages of the module docstring."""

    def __init__(self, block, num_frames: int, attn_impl: str = FAST_ATTN_IMPL,
                 cross_impl: str = FAST_CROSS_IMPL, pointwise_impl: str = FAST_POINTWISE_IMPL,
                 qkv_impl: str = FAST_QKV_IMPL):
        self.block = block
        self.num_frames = num_frames
        self.attn_impl = attn_impl
        self.cross_impl = cross_impl
        self.pointwise_impl = pointwise_impl
        self.qkv_impl = qkv_impl
        sa = block.self_attn
        if attn_impl == "hip":
            self.w_qkv, self.b_qkv = _pack_qkv(sa)

    def rows(self, e0):
        """The block's modulation rows per frame, [F, 6, C]: its modulation parameter plus the
        time projection e0 [1, F, 6, C] (models/fast_dit.py:275-276)."""
        blk = self.block
        return (blk.modulation.unsqueeze(0) + e0).reshape(self.num_frames, 6, blk.modulation.shape[-1])

    def __call__(self, x, e0, cos, sin, ck, cv, seqlen_k=None, h=None, next_stage=None):
        """x [B, L, C] bf16; e0 [1, F, 6, C] time projection; cos/sin [L, 64]; ck/cv the
        block's text keys/values [B, Lc, n, d]; seqlen_k: per-sample text lengths or None.

        Chained use (FastWanDiT): h is this block's norm1 + modulation output when the pass
        that ended the previous block already made it; next_stage = (rows, LayerNorm, shift,
        scale) of the stage that follows this block (the next block's norm1 + modulation, or
        the output head's), done in the same pass as this block's gated residual.  Then the
        call returns (x, h_next); otherwise x."""
        blk, nf = self.block, self.num_frames
        B, L, C = x.shape
        fused = self.pointwise_impl == "hip" and x.is_cuda
        stage = _hip_stage if fused else _eager_stage
        e = self.rows(e0)
        if fused:
            x = x.contiguous()
        if h is None:
            _, h = stage(x, None, e, nf, shift=0, scale=1, ln=blk.norm1)
        y = _linear(self._self_attention(h, cos, sin).reshape(B, L, C), blk.self_attn.o)
        x, h = stage(x, y, e, nf, gate=2, ln=blk.norm3)
        y = _linear(self._cross_attention(h, ck, cv, seqlen_k).reshape(B, L, C), blk.cross_attn.o)
        x, h = stage(x, y, e, nf, shift=3, scale=4, ln=blk.norm2)
        y = (_ffn_gelu_epilogue if fused else _ffn_eager)(h, blk.ffn)
        if next_stage is None:
            x, _ = stage(x, y, e, nf, gate=5, norm=False)
            return x
        mod, ln, shift, scale = next_stage
        return stage(x, y, e, nf, gate=5, shift=shift, scale=scale, ln=ln, mod=mod)

    def _self_attention(self, h, cos, sin):
        sa = self.block.self_attn
        B, L, C = h.shape
        heads = (B, L, sa.num_heads, sa.head_dim)
        scale = sa.head_dim ** -0.5
        if self.attn_impl == "hip":
            if self.qkv_impl == "hip":
                qkv, sumsq = ops.qkv_proj_sumsq(h.contiguous(), self.w_qkv, self.b_qkv, 2 * C)
                q, k, v = (t.view(heads) for t in qkv.split(C, dim=-1))
                return ops.self_attn_fused_sumsq(q, k, v, sumsq, sa.norm_q.weight, sa.norm_k.weight,
                                                 sa.norm_q.eps, cos, sin, scale)
            q, k, v = (t.view(heads) for t in F.linear(h, self.w_qkv, self.b_qkv).split(C, dim=-1))
            return ops.self_attn_fused(q, k, v, sa.norm_q.weight, sa.norm_k.weight, sa.norm_q.eps,
                                       cos, sin, scale)
        q = _rms_normalize(_linear(h, sa.q), sa.norm_q.weight, sa.norm_q.eps).view(heads)
        k = _rms_normalize(_linear(h, sa.k), sa.norm_k.weight, sa.norm_k.eps).view(heads)
        return _sdpa(_rope(q, cos, sin), _rope(k, cos, sin), _linear(h, sa.v).view(heads))

    def _cross_attention(self, h, ck, cv, seqlen_k):
        ca = self.block.cross_attn
        B, L, C = h.shape
        heads = (B, L, ca.num_heads, ca.head_dim)
        q = _linear(h, ca.q)
        if self.cross_impl == "hip":
            return ops.cross_attn_fused(q.view(heads), ck, cv, ca.norm_q.weight, ca.norm_q.eps,
                                        seqlen_k, ca.head_dim ** -0.5)
        q = _rms_normalize(q, ca.norm_q.weight, ca.norm_q.eps).view(heads)
        return _sdpa(q, ck, cv, None if seqlen_k is None else seqlen_k.tolist())


def cross_kv(block, context, impl: str = FAST_CROSS_IMPL):
    """The text keys and values one block attends to, [B, Lc, n, d] each: K RMS-normalised
    over all heads of a text token, V as projected.  Computed once per prompt and kept in
    HBM for every denoising step (the reference's _FastCrossKV, models/fast_dit.py:464-477)."""
    ca = block.cross_attn
    B, Lc, _ = context.shape
    heads = (B, Lc, ca.num_heads, ca.head_dim)
    k = _linear(context, ca.k)
    if impl == "hip":
        k = ops.rms_norm(k.view(heads), ca.norm_k.weight, ca.norm_k.eps)
    else:
        k = _rms_normalize(k, ca.norm_k.weight, ca.norm_k.eps).view(heads)
    return k, _linear(context, ca.v).view(heads)


class _FastCrossKV:
    """cross_kv() bound to one block (the reference's per-block callable)."""

    def __init__(self, block, cross_impl: str = FAST_CROSS_IMPL):
        self.block, self.cross_impl = block, cross_impl

    def __call__(self, context):
        return cross_kv(self.block, context, self.cross_impl)


def head_rows(head, e, frames):
    """The output head's modulation rows per frame, [F, 2, C] (shift, scale): its modulation
    parameter plus the time embedding e [1, F, C] (models/fast_dit.py:480-505)."""
    C = head.modulation.shape[-1]
    return (head.modulation.unsqueeze(0) + e.unsqueeze(2)).reshape(frames, 2, C)


def noise_prediction(head, x, e, grid, patch_size, out_dim, guide_scale, h=None):
    """Output head and CFG (the reference's _FastHead, models/fast_dit.py:480-505): the final
    tokens x [2, L, C] get the head's per-frame adaLN (modulation rows from the time
    embedding e [1, F, C]) and its projection to one patch of out_dim channels each; the
    patches go back to the latent grid [2, out_dim, F*pt, H*ph, W*pw]; batch row 0 is the
    cond and row 1 the uncond prediction, returned as uncond + guide (cond - uncond).
    h: the head's adaLN output when the last block's final pass already made it."""
    f, hh, ww = grid
    pt, ph, pw = patch_size
    if h is None:
        _, h = _eager_stage(x, None, head_rows(head, e, f), f, shift=0, scale=1, ln=head.norm)
    y = _linear(h, head.head)
    n = y.shape[0]
    # token (t, i, j) patch (a, b, c) channel o -> latent [o, t*pt + a, i*ph + b, j*pw + c]
    y = y.view(n, f, hh, ww, pt, ph, pw, out_dim).permute(0, 7, 1, 4, 2, 5, 3, 6)
    y = y.reshape(n, out_dim, f * pt, hh * ph, ww * pw).to(torch.bfloat16)
    cond, uncond = y[0], y[1]
    return uncond + guide_scale * (cond - uncond)


class FastWanDiT:
    """The whole DiT with batched CFG on one GPU (the reference's FastWanDiT,
    models/fast_dit.py:561-697).  Per prompt, set_context() embeds the two text contexts and
    precomputes every block's text K/V; per denoising step, calling the object with the
    latent [C, F, H, W] and the timestep returns the guided flow prediction [C, F, H, W]."""

    def __init__(self, model: WanModel, grid, guide_scale: float, attn_impl: str = FAST_ATTN_IMPL,
                 cross_impl: str = FAST_CROSS_IMPL, pointwise_impl: str = FAST_POINTWISE_IMPL):
        self.model = model
        self.grid = tuple(int(g) for g in grid)
        self.num_frames = self.grid[0]
        self.seq_len = math.prod(self.grid)
        self.guide_scale = guide_scale
        self.device = model.patch_embedding.weight.device
        head_dim = model.dim // model.num_heads
        self.cos, self.sin = _rope_mod.rope_tables(model.freqs, self.grid, head_dim, self.device)
        self.blocks = [_FastBlock(b, self.num_frames, attn_impl, cross_impl, pointwise_impl)
                       for b in model.blocks]
        self.cross_impl = cross_impl
        self.context = None
        self.seqlen_k = None

    def set_context(self, ctx_cond, ctx_null, context_lens: Optional[Sequence[int]] = None):
        """ctx_cond / ctx_null [1, Lc, text_dim]: the text embedding and every block's cross
        K/V, once per prompt.  context_lens: valid text tokens of (cond, uncond); None attends
        to all Lc tokens, as the reference pipeline does."""
        ctx = torch.cat([ctx_cond, ctx_null], dim=0).to(self.device, torch.bfloat16)
        text = self.model.text_embedding(ctx)
        self.context = [cross_kv(b, text, self.cross_impl) for b in self.model.blocks]
        self.seqlen_k = None if context_lens is None else \
            torch.tensor(list(context_lens), dtype=torch.int32, device=self.device)

    def time_rows(self, t):
        """Time conditioning per latent frame.  Frame 0 holds the conditioning image and is
        embedded at t = 0, the others at t.  Returns the head's embedding [1, F, C] and the
        blocks' modulation input [1, F, 6, C]."""
        m = self.model
        frame_t = float(t) * (torch.arange(self.num_frames) > 0).double()
        sincos = sinusoidal_embedding_1d(m.freq_dim, frame_t).to(torch.bfloat16)
        if self.device.type == "cuda":
            # through pinned memory without a wait: a copy from pageable memory would block
            # the host until the stream drained, once per denoising step
            sincos = sincos.pin_memory().to(self.device, non_blocking=True)
        else:
            sincos = sincos.to(self.device)
        emb = m.time_embedding(sincos.unsqueeze(0))
        return emb, m.time_projection(emb).view(1, self.num_frames, 6, m.dim)

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
        """One guided flow prediction.  The blocks are chained: the pass that ends block i
        (its gated residual) also makes block i+1's norm1 + modulation, and the last block's
        the output head's LayerNorm + modulation, so each block boundary is one pass over the
        residual stream instead of two (the same ops and roundings as separate stages)."""
        if self.context is None:
            raise RuntimeError("FastWanDiT: call set_context() before the first step")
        e, e0 = self.time_rows(t)
        x = self.patch(latent)
        m = self.model
        n = len(self.blocks)
        h = None
        for i, (blk, (ck, cv)) in enumerate(zip(self.blocks, self.context)):
            if i + 1 < n:
                nxt = self.blocks[i + 1]
                following = (nxt.rows(e0), nxt.block.norm1, 0, 1)
            else:
                following = (head_rows(m.head, e, self.num_frames), m.head.norm, 0, 1)
            x, h = blk(x, e0, self.cos, self.sin, ck, cv, self.seqlen_k, h=h, next_stage=following)
        return noise_prediction(m.head, x, e, self.grid, m.patch_size, m.out_dim, self.guide_scale, h=h)


def denoise(fast: FastWanDiT, latent: torch.Tensor, steps: int, shift: float,
            image_latent: Optional[torch.Tensor] = None, num_train_timesteps: int = 1000):
    """The TI2V denoising loop (inference_neuron_ti2v.py:448-531): the latent in bf16 as the
    reference keeps it, one DiT call and one UniPC step (on the device) per timestep; with
    `image_latent` [C, 1, H, W], frame 0 is the image latent before the first call and after
    every step (the mask2 blend).  Returns the final bf16 latent."""
    from .unipc import FlowUniPC
    sampler = FlowUniPC(num_train_timesteps=num_train_timesteps, shift=1.0)
    sampler.set_timesteps(steps, shift=shift)
    x = latent.to(torch.bfloat16)
    image = None if image_latent is None else image_latent.to(x.device, torch.bfloat16)
    if image is not None:
        x = x.clone()
        x[:, :1] = image
    for t in sampler.timesteps:
        x = sampler.step(fast(x, t), x)
        if image is not None:
            x[:, :1] = image
    return x
