"""CPU oracle of the Wan DiT attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only to check results against (or, for the CPU baseline, as the
thing timed on host cores).  The product path (wan2-ti2v-5b_amd) never calls it.

It restates, in plain torch-on-CPU (and numpy for the brute-force forms), the
reference's arithmetic for this path, with the reference's bf16 rounding points
when given bf16 tensors and without them when given fp32 tensors:

  rope_params        wan/modules/rope_neuron.py:14-24
  wan_freqs          wan/modules/model.py:396-403
  rope_tables        models/fast_dit.py:548-558
  rope               models/fast_dit.py:163-169
  rope_expanded      kernels/rope.py:39-71 (cos_expanded / sin_signed form)
  rms_qk             models/fast_dit.py:134-147 (TP=1: the all-reduce is the identity, :90-92)
  rms                models/fast_dit.py:156-160
  sdpa               models/fast_dit.py:186-189, keys limited to actual_seqlen_k as
                     kernels/self_attention_nst.py:73-78,715-722
  self_attn_path     models/fast_dit.py:281-292
  cross_attn_path    models/fast_dit.py:297-304
  brute_attention    scripts/validate/attn_bench.py:54-60 (per-head loop), float64 numpy
  block_forward      scripts/validate/ref_fp32.py:37-59 (one WanAttentionBlock, fp32)
  dit_forward        scripts/validate/ref_fp32.py:62-99 (CFG noise prediction, fp32)
  unpatchify         wan/modules/model.py:496-519
  adaln              models/fast_dit.py:172-181,280,294,306-311 with WanLayerNorm
                     (wan/modules/model.py:89-99): one bf16 adaLN stage of a block
  layer_norm64       float64 numpy LayerNorm (biased variance), what adaln is checked against

Each function is pinned by tests/test_oracle.py (closed forms, invariants,
library routines and float64 brute force); see that file's header.
"""
import math
from typing import Optional, Sequence

import numpy as np
import torch
import torch.nn.functional as F

HEAD_DIM = 128
DIM = 3072
NUM_HEADS = 24
EPS = 1e-6
THETA = 10000.0


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def rope_params(max_seq_len: int, dim: int, theta: float = THETA) -> torch.Tensor:
    """Angles [max_seq_len, dim//2] fp32: p * theta^(-2j/dim) (wan/modules/rope_neuron.py:14-24)."""
    return torch.outer(torch.arange(max_seq_len).float(),
                       1.0 / torch.pow(theta, torch.arange(0, dim, 2).float().div(dim)))


def wan_freqs(head_dim: int = HEAD_DIM, max_seq_len: int = 1024) -> torch.Tensor:
    """Frame/height/width angle table [1024, 64] (wan/modules/model.py:396-403): 44/42/42 dims."""
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


def rope_tables(freqs: torch.Tensor, grid: Sequence[int], head_dim: int = HEAD_DIM):
    """cos, sin [L, head_dim/2] fp32 for token index f*h*w + y*w + x (models/fast_dit.py:548-558)."""
    f, h, w = grid
    c = head_dim // 2
    fr = freqs.float().split([c - 2 * (c // 3), c // 3, c // 3], dim=1)
    ang = torch.cat([
        fr[0][:f].view(f, 1, 1, -1).expand(f, h, w, -1),
        fr[1][:h].view(1, h, 1, -1).expand(f, h, w, -1),
        fr[2][:w].view(1, 1, w, -1).expand(f, h, w, -1),
    ], dim=-1).reshape(f * h * w, c)
    return torch.cos(ang), torch.sin(ang)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation, fp32 math, cast back to x.dtype (models/fast_dit.py:163-169).

    x [B, L, n, d]; cos/sin [L, d/2].
    """
    B, L, n, d = x.shape
    cos = cos.view(1, L, 1, d // 2)
    sin = sin.view(1, L, 1, d // 2)
    xp = x.float().reshape(B, L, n, d // 2, 2)
    xr, xi = xp[..., 0], xp[..., 1]
    out = torch.stack([xr * cos - xi * sin, xr * sin + xi * cos], dim=-1)
    return out.reshape(B, L, n, d).to(x.dtype)


def rope_expanded(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """kernels/rope.py:39-71 form in float64: out = x*cos_exp + swap_pairs(x)*sin_signed.

    cos_exp[:, 2j] = cos_exp[:, 2j+1] = cos_j; sin_signed[:, 2j] = -sin_j, [:, 2j+1] = +sin_j
    (the table layout built by kernels/kernel_builder/rope.py:18-22).  x [L, n, d].
    """
    cos_exp = np.repeat(cos, 2, axis=-1)[:, None, :]
    sin_signed = np.repeat(sin, 2, axis=-1)
    sin_signed[:, 0::2] *= -1.0
    sin_signed = sin_signed[:, None, :]
    swap = np.empty_like(x)
    swap[..., 0::2] = x[..., 1::2]
    swap[..., 1::2] = x[..., 0::2]
    return x * cos_exp + swap * sin_signed


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def rms_qk(q: torch.Tensor, k: torch.Tensor, gamma_q: torch.Tensor, gamma_k: torch.Tensor,
           eps: float = EPS):
    """_tp_rms_qk at TP=1 (models/fast_dit.py:134-147).

    q [B, Lq, C], k [B, Lk, C]; RMS over all C channels of a token; fp32 statistics,
    `.type_as(x)` rounding, then `* gamma` in the tensors' dtype.
    """
    def one(x, g):
        xf = x.float()
        inv = torch.rsqrt(xf.pow(2).sum(-1, keepdim=True) / x.shape[-1] + eps)
        return (xf * inv).type_as(x) * g
    return one(q, gamma_q), one(k, gamma_k)


def rms(x: torch.Tensor, gamma: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """_tp_rms at TP=1 (models/fast_dit.py:156-160)."""
    xf = x.float()
    ss = xf.pow(2).sum(-1, keepdim=True)
    return (xf * torch.rsqrt(ss / x.shape[-1] + eps)).type_as(x) * gamma


def inv_rms(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """The per-token statistic 1/sqrt(mean(x^2) + eps), fp32 [B, L]."""
    xf = x.float()
    return torch.rsqrt(xf.pow(2).sum(-1) / x.shape[-1] + eps)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
         seqlen_k=None) -> torch.Tensor:
    """softmax(q k^T * scale) v over keys < seqlen_k[b] (models/fast_dit.py:186-189).

    q [B, Lq, n, d], k/v [B, Lk, n, d] -> [B, Lq, n, d], computed by torch's CPU
    SDPA in the inputs' dtype.  seqlen_k: None (all keys), an int, or one length
    per sample; keys at or beyond it are excluded (kernels/self_attention_nst.py:73-78).
    """
    B, Lk = k.shape[0], k.shape[1]
    if seqlen_k is None:
        lens = [Lk] * B
    elif isinstance(seqlen_k, int):
        lens = [seqlen_k] * B
    else:
        lens = [int(x) for x in seqlen_k]
    outs = []
    for b in range(B):
        n = lens[b]
        qb = q[b:b + 1].transpose(1, 2)
        kb = k[b:b + 1, :n].transpose(1, 2)
        vb = v[b:b + 1, :n].transpose(1, 2)
        if n == 0:
            outs.append(torch.zeros_like(q[b:b + 1]))
            continue
        ob = F.scaled_dot_product_attention(qb, kb, vb, scale=scale)
        outs.append(ob.transpose(1, 2))
    return torch.cat(outs, dim=0)


def brute_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: Optional[float] = None,
                    seqlen_k=None) -> np.ndarray:
    """float64 per-(batch, head) softmax loop (scripts/validate/attn_bench.py:54-60)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Lq, n, d = q.shape
    Lk = k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    lens = [Lk] * B if seqlen_k is None else (
        [int(seqlen_k)] * B if np.isscalar(seqlen_k) else [int(x) for x in seqlen_k])
    out = np.zeros((B, Lq, n, d))
    for b in range(B):
        m = lens[b]
        if m == 0:
            continue
        for h in range(n):
            s = q[b, :, h] @ k[b, :m, h].T * scale
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, h] = p @ v[b, :m, h]
    return out


def self_attn_path(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma_q: torch.Tensor,
                   gamma_k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   eps: float = EPS, scale: Optional[float] = None) -> torch.Tensor:
    """QK-RMSNorm -> RoPE -> SDPA, models/fast_dit.py:281-292.  q,k,v [B, L, n, d]."""
    B, L, n, d = q.shape
    qn, kn = rms_qk(q.reshape(B, L, n * d), k.reshape(B, L, n * d), gamma_q, gamma_k, eps)
    qr = rope(qn.view(B, L, n, d), cos, sin)
    kr = rope(kn.view(B, L, n, d), cos, sin)
    return sdpa(qr, kr, v, scale=scale)


def cross_attn_path(q: torch.Tensor, ck: torch.Tensor, cv: torch.Tensor, gamma_q: torch.Tensor,
                    eps: float = EPS, seqlen_k=None, scale: Optional[float] = None) -> torch.Tensor:
    """Cross Q-RMSNorm -> SDPA over the text keys, models/fast_dit.py:297-304."""
    B, Lq, n, d = q.shape
    qn = rms(q.reshape(B, Lq, n * d), gamma_q, eps).view(B, Lq, n, d)
    return sdpa(qn, ck, cv, scale=scale, seqlen_k=seqlen_k)


def rel_rms(y: torch.Tensor, ref: torch.Tensor) -> float:
    """||y - ref||_2 / ||ref||_2 (scripts/validate/attn_bench.py:114-115)."""
    y = y.double()
    ref = ref.double()
    return float((y - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt())


# ---------------------------------------------------------------------------
# block and DiT forward in fp32 (scripts/validate/ref_fp32.py:20-109)
# ---------------------------------------------------------------------------

def _rms32(x, norm):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + norm.eps) * norm.weight.float()


def _lin32(x, m):
    return F.linear(x, m.weight.float(), None if m.bias is None else m.bias.float())


def _ln32(x, ln):
    w = None if ln.weight is None else ln.weight.float()
    b = None if ln.bias is None else ln.bias.float()
    return F.layer_norm(x, (x.shape[-1],), w, b, eps=ln.eps)


def block_forward(blk, x, e0, cos, sin, ck, cv, num_frames):
    """One WanAttentionBlock in fp32 with exact SDPA (ref_fp32.py:37-59).

    blk: a module with the WanAttentionBlock parameter names; x [B, L, C]; e0 [1, F, 6, C];
    cos/sin [L, d/2]; ck/cv [B, Lc, n, d].  All arithmetic in fp32.
    """
    sa, ca = blk.self_attn, blk.cross_attn
    B, L, C = x.shape
    n, d = sa.num_heads, sa.head_dim
    x = x.float()
    e = [t.squeeze(2) for t in (blk.modulation.float().unsqueeze(0) + e0.float()).chunk(6, dim=2)]

    def per_frame(t):
        return t.view(B, num_frames, L // num_frames, C)

    def mod(h, shift, scale):
        return (per_frame(h) * (1 + scale.unsqueeze(2)) + shift.unsqueeze(2)).view(B, L, C)

    def gate(y, g):
        return (per_frame(y) * g.unsqueeze(2)).view(B, L, C)

    def attn(q, k, v):
        q, k, v = (t_.transpose(1, 2).contiguous() for t_ in (q, k, v))
        return F.scaled_dot_product_attention(q, k, v).transpose(1, 2)

    h = mod(_ln32(x, blk.norm1), e[0], e[1])
    q = rope(_rms32(_lin32(h, sa.q), sa.norm_q).view(B, L, n, d), cos, sin)
    k = rope(_rms32(_lin32(h, sa.k), sa.norm_k).view(B, L, n, d), cos, sin)
    v = _lin32(h, sa.v).view(B, L, n, d)
    x = x + gate(_lin32(attn(q, k, v).reshape(B, L, C), sa.o), e[2])
    h = _ln32(x, blk.norm3)
    q = _rms32(_lin32(h, ca.q), ca.norm_q).view(B, L, n, d)
    x = x + _lin32(attn(q, ck.float(), cv.float()).reshape(B, L, C), ca.o)
    h = mod(_ln32(x, blk.norm2), e[3], e[4])
    y = _lin32(F.gelu(_lin32(h, blk.ffn[0]), approximate="tanh"), blk.ffn[2])
    return x + gate(y, e[5])


def sinusoidal_embedding_1d(dim: int, position: torch.Tensor) -> torch.Tensor:
    """wan/modules/model.py:15-25, float64."""
    half = dim // 2
    position = position.type(torch.float64)
    s = torch.outer(position, torch.pow(10000, -torch.arange(half).to(position).div(half)))
    return torch.cat([torch.cos(s), torch.sin(s)], dim=1)


def text_context(tx, ctx):
    """The DiT's text embedding `tx` (a Sequential: Linear(text_dim -> dim), tanh-GELU,
    Linear) in fp32 (wan/modules/model.py:469-475; ref_fp32.py:72-73)."""
    return _lin32(F.gelu(_lin32(ctx.float(), tx[0]), approximate="tanh"), tx[2])


def cross_kv(blk, context, heads, d):
    """One block's cross-attention keys and values in fp32: K = RMSNorm over all heads of a
    text token (norm_k), V as projected, each [B, Lc, heads, d] (models/fast_dit.py:464-477)."""
    ca = blk.cross_attn
    B = context.shape[0]
    ck = _rms32(_lin32(context, ca.k), ca.norm_k).view(B, -1, heads, d)
    cv = _lin32(context, ca.v).view(B, -1, heads, d)
    return ck, cv


def dit_forward(model, latent, t, ctx_cond, ctx_null, grid, guide_scale):
    """CFG noise prediction of the whole DiT in fp32 (ref_fp32.py:62-99): latent [C, F, H, W],
    contexts [1, Lc, text_dim] -> [C_out, F, H, W].

    Runs on the device that holds the model's (fp32) weights; the RoPE tables, the
    sinusoidal time embedding and the patch-embedding convolution are computed on the host
    and moved there."""
    f, h, w = grid
    L = f * h * w
    dim, heads = model.dim, model.num_heads
    d = dim // heads
    dev = model.head.head.weight.device
    cos, sin = (t_.to(dev) for t_ in rope_tables(model.freqs, grid, d))
    t_frames = torch.full((f,), float(t), dtype=torch.float64)
    t_frames[0] = 0.0
    te = model.time_embedding
    s = sinusoidal_embedding_1d(model.freq_dim, t_frames).float().to(dev)
    e = _lin32(F.silu(_lin32(s, te[0])), te[2])
    e = e.unsqueeze(0)                                              # [1, F, C]
    e0 = _lin32(F.silu(e), model.time_projection[1]).unflatten(2, (6, dim))
    context = text_context(model.text_embedding, torch.cat([ctx_cond, ctx_null], 0).float().to(dev))
    pe = model.patch_embedding
    x = F.conv3d(latent.float().cpu().unsqueeze(0), pe.weight.float().cpu(), pe.bias.float().cpu(),
                 stride=pe.stride).to(dev)
    x = x.flatten(2).transpose(1, 2).expand(2, -1, -1).contiguous()
    for blk in model.blocks:
        ck, cv = cross_kv(blk, context, heads, d)
        x = block_forward(blk, x, e0, cos, sin, ck, cv, f)
    hd = model.head
    m = [t_.squeeze(2) for t_ in (hd.modulation.float().unsqueeze(0) + e.unsqueeze(2)).chunk(2, dim=2)]
    xn = _ln32(x, hd.norm).view(2, f, L // f, dim)
    y = _lin32((xn * (1 + m[1].unsqueeze(2)) + m[0].unsqueeze(2)).view(2, L, dim), hd.head)
    y = unpatchify(y, grid, model.patch_size, model.out_dim)
    return y[1] + guide_scale * (y[0] - y[1])


def unpatchify(y, grid, patch_size, c):
    """[B, f*h*w, p*q*r*c] -> [B, c, f*p, h*q, w*r], einsum 'fhwpqrc->cfphqwr'
    (wan/modules/model.py:512-518)."""
    f, h, w = grid
    p, q, r = patch_size
    B = y.shape[0]
    return y.view(B, f, h, w, p, q, r, c).permute(0, 7, 1, 4, 2, 5, 3, 6).reshape(B, c, f * p, h * q, w * r)


def adaln(x: torch.Tensor, y: Optional[torch.Tensor] = None, e: Optional[torch.Tensor] = None,
          frames: int = 1, gate_idx: int = -1, shift_idx: int = -1, scale_idx: int = -1,
          ln_weight: Optional[torch.Tensor] = None, ln_bias: Optional[torch.Tensor] = None,
          eps: float = EPS, norm: bool = True):
    """One adaLN stage of a WanAttentionBlock with the reference's bf16 rounding points,
    as torch CPU ops in the order the reference's eager graph runs them:

      x + _gate(y, e[gate])          models/fast_dit.py:294,311 (_gate :179-181), or x + y (:306)
      WanLayerNorm(r)                wan/modules/model.py:89-99: F.layer_norm on bf16 input
      _modulate(ln, e[shift], e[scale])   models/fast_dit.py:172-177, :280,307

    x, y [B, L, C]; e [frames, 6, C] (block modulation + per-frame time projection).
    Returns (r, h) with h None when norm is False."""
    x = x.bfloat16()
    B, L, C = x.shape

    def rows(i):
        return e[:, i].bfloat16().unsqueeze(0)          # [1, F, C]

    def per_frame(t):
        return t.view(B, frames, L // frames, C)

    r = x
    if y is not None:
        y = y.bfloat16()
        if gate_idx >= 0:
            y = (per_frame(y) * rows(gate_idx).unsqueeze(2)).view(B, L, C)
        r = x + y
    if not norm:
        return r, None
    w = None if ln_weight is None else ln_weight.bfloat16()
    b = None if ln_bias is None else ln_bias.bfloat16()
    h = F.layer_norm(r, (C,), w, b, eps)
    if shift_idx >= 0:
        h = (per_frame(h) * (1 + rows(scale_idx).unsqueeze(2)) + rows(shift_idx).unsqueeze(2)).view(B, L, C)
    return r, h


def layer_norm64(x: np.ndarray, w: Optional[np.ndarray] = None, b: Optional[np.ndarray] = None,
                 eps: float = EPS) -> np.ndarray:
    """LayerNorm over the last axis in float64: (x - mean) / sqrt(var + eps) [* w + b], with
    the biased variance torch.nn.LayerNorm uses."""
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    out = (x - mu) / np.sqrt(var + eps)
    if w is not None:
        out = out * np.asarray(w, dtype=np.float64) + np.asarray(b, dtype=np.float64)
    return out
