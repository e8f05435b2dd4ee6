"""torch operators over the C ABI (torch.library custom ops with fake kernels).

Every op takes bf16 CUDA tensors in the DiT projection layout [B, L, H, 128]
(views of [B, L, 3072] are accepted as they are: only the head_dim axis must be
contiguous), launches on torch's current stream of the tensor's device and
returns a new contiguous [B, Lq, H, 128] tensor.  Outputs and workspaces come
from torch's caching allocator; the native side allocates nothing.

The fake (meta) kernels let torch.compile trace the ops without running them.
"""
from typing import Optional, Tuple

import torch

from . import _native as N

HEAD_DIM = 128


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check4(name: str, x: torch.Tensor) -> None:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(x).__name__}")
    if x.dim() != 4:
        raise ValueError(f"{name}: expected [B, L, H, {HEAD_DIM}], got shape {tuple(x.shape)}")
    if x.shape[-1] != HEAD_DIM:
        raise ValueError(f"{name}: head_dim must be {HEAD_DIM}, got {x.shape[-1]}")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected bfloat16, got {x.dtype}")
    if x.device.type != "cuda":
        raise ValueError(f"{name}: expected a CUDA (HIP) tensor, got device {x.device}")
    if x.numel() == 0:
        return
    if x.stride(-1) != 1:
        raise ValueError(f"{name}: the head_dim axis must be contiguous (stride {x.stride(-1)})")
    if any(s % 8 for s in x.stride()[:3]) or x.data_ptr() % 16:
        raise ValueError(f"{name}: strides {x.stride()} must be multiples of 8 elements "
                         "and the data 16-byte aligned")


def _check_qkv(fn: str, q, k, v):
    _check4(f"{fn}: q", q)
    _check4(f"{fn}: k", k)
    _check4(f"{fn}: v", v)
    if k.shape != v.shape:
        raise ValueError(f"{fn}: k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"{fn}: q {tuple(q.shape)} and k {tuple(k.shape)} disagree on batch/heads")
    if not (q.device == k.device == v.device):
        raise ValueError(f"{fn}: q, k, v are on different devices")


def _check_vec(fn: str, name: str, t: torch.Tensor, n: int, dtype, device) -> None:
    if t.device != device or t.dtype != dtype or t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{fn}: {name} must be a contiguous {dtype} tensor of {n} elements on "
                         f"{device}, got {t.dtype} {tuple(t.shape)} on {t.device}")


def _check_rope(fn: str, cos: torch.Tensor, sin: torch.Tensor, L: int, device) -> None:
    for name, t in (("cos", cos), ("sin", sin)):
        if t.device != device or t.dtype != torch.float32 or not t.is_contiguous() \
                or t.numel() != L * HEAD_DIM // 2:
            raise ValueError(f"{fn}: {name} must be a contiguous float32 [{L}, {HEAD_DIM // 2}] "
                             f"tensor on {device}, got {t.dtype} {tuple(t.shape)} on {t.device}")


def _seqlen_ptr(fn: str, seqlen_k: Optional[torch.Tensor], B: int, device) -> int:
    if seqlen_k is None:
        return 0
    _check_vec(fn, "seqlen_k", seqlen_k, B, torch.int32, device)
    return seqlen_k.data_ptr()


# ---------------------------------------------------------------------------
# self-attention (kernels/self_attention_nst.py:49-117; models/fast_dit.py:186-207)
# ---------------------------------------------------------------------------

@torch.library.custom_op("wan_hip::flash_self_attn", mutates_args=())
def flash_self_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    softmax_scale: float, actual_seqlen_k: int) -> torch.Tensor:
    fn = "flash_self_attn"
    _check_qkv(fn, q, k, v)
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    if actual_seqlen_k > Lk:
        raise ValueError(f"{fn}: actual_seqlen_k must be in (0, {Lk}], got {actual_seqlen_k}")
    out = torch.empty((B, Lq, H, D), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        N.check("wan_flash_self_attn", N.lib().wan_flash_self_attn(
            N.tensor4(q), N.tensor4(k), N.tensor4(v), N.tensor4(out), B, H, Lq, Lk, D,
            float(softmax_scale), int(actual_seqlen_k), _stream(q.device)))
    return out


@flash_self_attn.register_fake
def _(q, k, v, softmax_scale, actual_seqlen_k):
    return q.new_empty(q.shape)


@torch.library.custom_op("wan_hip::cross_attn", mutates_args=())
def cross_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               seqlen_k: Optional[torch.Tensor], softmax_scale: float) -> torch.Tensor:
    fn = "cross_attn"
    _check_qkv(fn, q, k, v)
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    sk = _seqlen_ptr(fn, seqlen_k, B, q.device)
    out = torch.empty((B, Lq, H, D), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        N.check("wan_cross_attn", N.lib().wan_cross_attn(
            N.tensor4(q), N.tensor4(k), N.tensor4(v), N.tensor4(out), B, H, Lq, Lk, D,
            float(softmax_scale), sk, _stream(q.device)))
    return out


@cross_attn.register_fake
def _(q, k, v, seqlen_k, softmax_scale):
    return q.new_empty(q.shape)


# ---------------------------------------------------------------------------
# fused spans of _FastBlock.forward (models/fast_dit.py:281-292 and :297-304)
# ---------------------------------------------------------------------------

@torch.library.custom_op("wan_hip::self_attn_fused", mutates_args=())
def self_attn_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    gamma_q: torch.Tensor, gamma_k: torch.Tensor, eps: float,
                    cos: torch.Tensor, sin: torch.Tensor, softmax_scale: float) -> torch.Tensor:
    fn = "self_attn_fused"
    _check_qkv(fn, q, k, v)
    B, L, H, D = q.shape
    if k.shape[1] != L:
        raise ValueError(f"{fn}: self-attention needs Lq == Lk, got {L} and {k.shape[1]}")
    _check_vec(fn, "gamma_q", gamma_q, H * D, torch.bfloat16, q.device)
    _check_vec(fn, "gamma_k", gamma_k, H * D, torch.bfloat16, q.device)
    _check_rope(fn, cos, sin, L, q.device)
    lib = N.lib()
    ws = torch.empty(max(1, lib.wan_self_attn_fused_workspace(B, H, L)), dtype=torch.uint8,
                     device=q.device)
    out = torch.empty((B, L, H, D), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        N.check("wan_self_attn_fused", lib.wan_self_attn_fused(
            N.tensor4(q), N.tensor4(k), N.tensor4(v), N.tensor4(out), B, H, L, D,
            gamma_q.data_ptr(), gamma_k.data_ptr(), float(eps), cos.data_ptr(), sin.data_ptr(),
            float(softmax_scale), ws.data_ptr(), ws.numel(), _stream(q.device)))
    return out


@self_attn_fused.register_fake
def _(q, k, v, gamma_q, gamma_k, eps, cos, sin, softmax_scale):
    return q.new_empty(q.shape)


@torch.library.custom_op("wan_hip::cross_attn_fused", mutates_args=())
def cross_attn_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma_q: torch.Tensor,
                     eps: float, seqlen_k: Optional[torch.Tensor],
                     softmax_scale: float) -> torch.Tensor:
    fn = "cross_attn_fused"
    _check_qkv(fn, q, k, v)
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    _check_vec(fn, "gamma_q", gamma_q, H * D, torch.bfloat16, q.device)
    sk = _seqlen_ptr(fn, seqlen_k, B, q.device)
    lib = N.lib()
    ws = torch.empty(max(1, lib.wan_cross_attn_fused_workspace(B, H, Lq)), dtype=torch.uint8,
                     device=q.device)
    out = torch.empty((B, Lq, H, D), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        N.check("wan_cross_attn_fused", lib.wan_cross_attn_fused(
            N.tensor4(q), N.tensor4(k), N.tensor4(v), N.tensor4(out), B, H, Lq, Lk, D,
            gamma_q.data_ptr(), float(eps), float(softmax_scale), sk, ws.data_ptr(), ws.numel(),
            _stream(q.device)))
    return out


@cross_attn_fused.register_fake
def _(q, k, v, gamma_q, eps, seqlen_k, softmax_scale):
    return q.new_empty(q.shape)


# ---------------------------------------------------------------------------
# standalone RoPE and RMSNorm (models/fast_dit.py:163-169, :156-160; kernels/rope.py:39-71)
# ---------------------------------------------------------------------------

@torch.library.custom_op("wan_hip::rope", mutates_args=())
def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    fn = "rope"
    _check4(f"{fn}: x", x)
    B, L, H, D = x.shape
    _check_rope(fn, cos, sin, L, x.device)
    out = torch.empty((B, L, H, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        N.check("wan_rope", N.lib().wan_rope(N.tensor4(x), out.data_ptr(), B, L, H, D,
                                             cos.data_ptr(), sin.data_ptr(), _stream(x.device)))
    return out


@rope.register_fake
def _(x, cos, sin):
    return x.new_empty(x.shape)


def _rms_call(x, gamma, eps, cos, sin, out, inv):
    B, L, H, D = x.shape
    with torch.cuda.device(x.device):
        N.check("wan_rms_norm", N.lib().wan_rms_norm(
            N.tensor4(x), None if out is None else out.data_ptr(), B, L, H, D,
            None if gamma is None else gamma.data_ptr(), float(eps),
            None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
            None if inv is None else inv.data_ptr(), _stream(x.device)))


@torch.library.custom_op("wan_hip::rms_norm", mutates_args=())
def rms_norm(x: torch.Tensor, gamma: torch.Tensor, eps: float,
             cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None) -> torch.Tensor:
    """_tp_rms over all H*128 channels of each token (optionally followed by _rope)."""
    fn = "rms_norm"
    _check4(f"{fn}: x", x)
    B, L, H, D = x.shape
    _check_vec(fn, "gamma", gamma, H * D, torch.bfloat16, x.device)
    if (cos is None) != (sin is None):
        raise ValueError(f"{fn}: give both cos and sin, or neither")
    if cos is not None:
        _check_rope(fn, cos, sin, L, x.device)
    out = torch.empty((B, L, H, D), dtype=x.dtype, device=x.device)
    _rms_call(x, gamma, eps, cos, sin, out, None)
    return out


@rms_norm.register_fake
def _(x, gamma, eps, cos=None, sin=None):
    return x.new_empty(x.shape)


@torch.library.custom_op("wan_hip::rms_inv", mutates_args=())
def rms_inv(x: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-token 1/rms over all H*128 channels, fp32 [B, L] (the statistic of _tp_rms)."""
    _check4("rms_inv: x", x)
    B, L = x.shape[:2]
    inv = torch.empty((B, L), dtype=torch.float32, device=x.device)
    _rms_call(x, None, eps, None, None, None, inv)
    return inv


@rms_inv.register_fake
def _(x, eps):
    return x.new_empty(x.shape[:2], dtype=torch.float32)


@torch.library.custom_op("wan_hip::flash_attn_qnorm", mutates_args=())
def flash_attn_qnorm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, inv_rms_q: torch.Tensor,
                     gamma_q: torch.Tensor, cos: Optional[torch.Tensor], sin: Optional[torch.Tensor],
                     seqlen_k: Optional[torch.Tensor], softmax_scale: float) -> torch.Tensor:
    """Attention with the query RMSNorm (and RoPE when cos/sin are given) applied in the kernel."""
    fn = "flash_attn_qnorm"
    _check_qkv(fn, q, k, v)
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    _check_vec(fn, "inv_rms_q", inv_rms_q, B * Lq, torch.float32, q.device)
    _check_vec(fn, "gamma_q", gamma_q, H * D, torch.bfloat16, q.device)
    if (cos is None) != (sin is None):
        raise ValueError(f"{fn}: give both cos and sin, or neither")
    if cos is not None:
        _check_rope(fn, cos, sin, Lq, q.device)
    sk = _seqlen_ptr(fn, seqlen_k, B, q.device)
    out = torch.empty((B, Lq, H, D), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        N.check("wan_flash_attn_qnorm", N.lib().wan_flash_attn_qnorm(
            N.tensor4(q), N.tensor4(k), N.tensor4(v), N.tensor4(out), B, H, Lq, Lk, D,
            inv_rms_q.data_ptr(), gamma_q.data_ptr(),
            None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
            float(softmax_scale), sk, _stream(q.device)))
    return out


@flash_attn_qnorm.register_fake
def _(q, k, v, inv_rms_q, gamma_q, cos, sin, seqlen_k, softmax_scale):
    return q.new_empty(q.shape)


# ─── adaLN: the pointwise stages of a WanAttentionBlock ─────────────────────

def _check_rows(fn: str, name: str, t: torch.Tensor, shape, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{fn}: {name} must be a tensor, got {type(t).__name__}")
    if t.dtype != torch.bfloat16 or t.device != device or tuple(t.shape) != tuple(shape) \
            or not t.is_contiguous() or (t.numel() and t.data_ptr() % 16):
        raise ValueError(f"{fn}: {name} must be a contiguous, 16-byte aligned bf16 tensor of shape "
                         f"{tuple(shape)} on {device}, got {t.dtype} {tuple(t.shape)} on {t.device}")


@torch.library.custom_op("wan_hip::adaln", mutates_args=())
def adaln_stage(x: torch.Tensor, y: Optional[torch.Tensor], e: Optional[torch.Tensor], frames: int,
                gate_idx: int, shift_idx: int, scale_idx: int, ln_weight: Optional[torch.Tensor],
                ln_bias: Optional[torch.Tensor], eps: float, norm: bool,
                e_mod: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """One fused adaLN stage (see adaln()).  Returns (x_out, h); x_out is empty when y is
    None and h is empty when norm is False."""
    fn = "adaln"
    if not isinstance(x, torch.Tensor) or x.dim() != 3:
        raise ValueError(f"{fn}: x must be a [B, L, C] tensor")
    B, L, C = x.shape
    if x.device.type != "cuda":
        raise ValueError(f"{fn}: expected a CUDA (HIP) tensor, got device {x.device}")
    _check_rows(fn, "x", x, (B, L, C), x.device)
    if y is not None:
        _check_rows(fn, "y", y, (B, L, C), x.device)
    if e is not None:
        _check_rows(fn, "e", e, (frames, 6, C), x.device)
    mod_rows = 6
    if e_mod is not None:
        if e_mod.dim() != 3 or not 1 <= e_mod.shape[1] <= 6:
            raise ValueError(f"{fn}: e_mod must be [frames, rows <= 6, C], got {tuple(e_mod.shape)}")
        mod_rows = e_mod.shape[1]
        _check_rows(fn, "e_mod", e_mod, (frames, mod_rows, C), x.device)
    if ln_weight is not None or ln_bias is not None:
        if ln_weight is None or ln_bias is None:
            raise ValueError(f"{fn}: give the LayerNorm weight and bias together")
        _check_rows(fn, "ln_weight", ln_weight, (C,), x.device)
        _check_rows(fn, "ln_bias", ln_bias, (C,), x.device)
    x_out = torch.empty_like(x) if y is not None else x.new_empty((0,))
    h = torch.empty_like(x) if norm else x.new_empty((0,))
    with torch.cuda.device(x.device):
        N.check("wan_adaln_ex", N.lib().wan_adaln_ex(
            x.data_ptr(), None if y is None else y.data_ptr(),
            None if y is None else x_out.data_ptr(), h.data_ptr() if norm else None,
            B, L, C, None if e is None else e.data_ptr(), int(frames), int(gate_idx),
            None if e_mod is None else e_mod.data_ptr(), mod_rows, int(shift_idx), int(scale_idx),
            None if ln_weight is None else ln_weight.data_ptr(),
            None if ln_bias is None else ln_bias.data_ptr(), float(eps), _stream(x.device)))
    return x_out, h


@adaln_stage.register_fake
def _(x, y, e, frames, gate_idx, shift_idx, scale_idx, ln_weight, ln_bias, eps, norm, e_mod=None):
    x_out = x.new_empty(x.shape) if y is not None else x.new_empty((0,))
    h = x.new_empty(x.shape) if norm else x.new_empty((0,))
    return x_out, h


def adaln(x: torch.Tensor, y: Optional[torch.Tensor] = None, e: Optional[torch.Tensor] = None,
          frames: int = 1, gate_idx: int = -1, shift_idx: int = -1, scale_idx: int = -1,
          ln_weight: Optional[torch.Tensor] = None, ln_bias: Optional[torch.Tensor] = None,
          eps: float = 1e-6, norm: bool = True, e_mod: Optional[torch.Tensor] = None):
    """The pointwise work of one WanAttentionBlock stage (models/fast_dit.py:280,294,306-311),
    on x [B, L, C] bf16 with the block's modulation rows e [frames, 6, C]:

        r = x  |  bf16(x + y)  |  bf16(x + bf16(y * e[f, gate_idx]))
        h = bf16(LayerNorm(r) [* w + b])  [then bf16(bf16(h * bf16(1 + m[f, scale_idx])) + m[f, shift_idx])]

    with m = e, or e_mod [frames, rows, C] when the shift and scale belong to another row set
    (the next block's, or the output head's two rows).  Returns (r, h); h is None when norm
    is False."""
    r, h = adaln_stage(x, y, e, frames, gate_idx, shift_idx, scale_idx, ln_weight, ln_bias, eps, norm,
                       e_mod)
    return (x if y is None else r), (h if norm else None)


# ─── the q/k/v projection with the QK-RMSNorm statistics in its epilogue ───────

@torch.library.custom_op("wan_hip::qkv_proj_sumsq", mutates_args=())
def qkv_proj_sumsq(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                   sq_cols: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """out = bf16(x weight^T + bias) for x [B, L, C] and an nn.Linear weight [N, C], with
    sumsq [sq_cols / 64, B * L] fp32: each token's sum of squares of bf16(out) over every
    64 of the first sq_cols columns (wan_qkv_proj_sumsq)."""
    fn = "qkv_proj_sumsq"
    if x.dim() != 3:
        raise ValueError(f"{fn}: x must be [B, L, C], got {tuple(x.shape)}")
    B, L, C = x.shape
    Nn = weight.shape[0]
    _check_rows(fn, "x", x, (B, L, C), x.device)
    _check_rows(fn, "weight", weight, (Nn, C), x.device)
    _check_rows(fn, "bias", bias, (Nn,), x.device)
    out = torch.empty((B, L, Nn), dtype=x.dtype, device=x.device)
    sumsq = torch.empty((max(sq_cols // 64, 1), B * L), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        N.check("wan_qkv_proj_sumsq", N.lib().wan_qkv_proj_sumsq(
            x.data_ptr(), weight.data_ptr(), bias.data_ptr(), out.data_ptr(), sumsq.data_ptr(),
            B * L, Nn, C, C, C, Nn, int(sq_cols), _stream(x.device)))
    return out, sumsq


@qkv_proj_sumsq.register_fake
def _(x, weight, bias, sq_cols):
    B, L, _ = x.shape
    return (x.new_empty((B, L, weight.shape[0])),
            x.new_empty((max(sq_cols // 64, 1), B * L), dtype=torch.float32))


@torch.library.custom_op("wan_hip::self_attn_fused_sumsq", mutates_args=())
def self_attn_fused_sumsq(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sumsq: torch.Tensor,
                          gamma_q: torch.Tensor, gamma_k: torch.Tensor, eps: float,
                          cos: torch.Tensor, sin: torch.Tensor, softmax_scale: float) -> torch.Tensor:
    """self_attn_fused with the QK-RMSNorm statistics from qkv_proj_sumsq (sumsq
    [4 H, B L]: q's 64-column partials, then k's): the q statistics pass disappears and
    the k pass reads k only to normalise and rotate it (wan_rms_norm_qk_sumsq)."""
    fn = "self_attn_fused_sumsq"
    _check_qkv(fn, q, k, v)
    B, L, H, D = q.shape
    if k.shape[1] != L:
        raise ValueError(f"{fn}: self-attention needs Lq == Lk, got {L} and {k.shape[1]}")
    _check_vec(fn, "gamma_q", gamma_q, H * D, torch.bfloat16, q.device)
    _check_vec(fn, "gamma_k", gamma_k, H * D, torch.bfloat16, q.device)
    _check_vec(fn, "sumsq", sumsq, 4 * H * B * L, torch.float32, q.device)
    _check_rope(fn, cos, sin, L, q.device)
    lib = N.lib()
    inv = torch.empty(B * L, dtype=torch.float32, device=q.device)
    khat = torch.empty((B, L, H, D), dtype=q.dtype, device=q.device)
    out = torch.empty((B, L, H, D), dtype=q.dtype, device=q.device)
    s = _stream(q.device)
    with torch.cuda.device(q.device):
        N.check("wan_rms_norm_qk_sumsq", lib.wan_rms_norm_qk_sumsq(
            N.tensor4(k), khat.data_ptr(), B, L, H, D, gamma_k.data_ptr(), float(eps),
            cos.data_ptr(), sin.data_ptr(), sumsq.data_ptr(), inv.data_ptr(), s))
        N.check("wan_flash_attn_qnorm", lib.wan_flash_attn_qnorm(
            N.tensor4(q), N.tensor4(khat), N.tensor4(v), N.tensor4(out), B, H, L, L, D,
            inv.data_ptr(), gamma_q.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            float(softmax_scale), None, s))
    return out


@self_attn_fused_sumsq.register_fake
def _(q, k, v, sumsq, gamma_q, gamma_k, eps, cos, sin, softmax_scale):
    return q.new_empty(q.shape)
