"""Pins the CPU oracle (oracle/ref.py) before any GPU result is compared with it.

Every oracle function is checked against something it does not share code with:
  * the float64 known-answer vectors of tests/golden/attn_golden.npz (independent numpy);
  * float64 brute force (scripts/validate/attn_bench.py:54-60 loop) on tiny shapes;
  * closed forms and invariants: RMSNorm of a constant row, scale invariance,
    RoPE identity at position 0, pair-norm preservation, the relative-position
    property, the kernels/rope.py expanded-table form, the angle formula;
  * masking special cases: len = Lk equals unmasked, len = 1 returns v[0],
    keys beyond len do not matter.
The last group plants plausible mistakes in copies of the oracle and shows that
the same checks reject each of them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ref

D = 128


def _r(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


# ---------------------------------------------------------------------------
# reusable checks (also applied to the planted mutants below)
# ---------------------------------------------------------------------------

def check_attention_vs_brute(attn_fn, seed=0):
    q, k, v = _r((2, 9, 3, D), seed), _r((2, 13, 3, D), seed + 1), _r((2, 13, 3, D), seed + 2)
    got = attn_fn(q, k, v).double().numpy()
    want = ref.brute_attention(q.numpy(), k.numpy(), v.numpy())
    return np.abs(got - want).max() < 1e-5


def check_mask(attn_fn, seed=0):
    q, k, v = _r((2, 7, 2, D), seed), _r((2, 11, 2, D), seed + 1), _r((2, 11, 2, D), seed + 2)
    lens = [4, 11]
    got = attn_fn(q, k, v, seqlen_k=lens)
    want = ref.brute_attention(q.numpy(), k.numpy(), v.numpy(), seqlen_k=lens)
    return np.abs(got.double().numpy() - want).max() < 1e-5


def check_rope_golden(rope_fn, tables_fn, golden):
    grid = tuple(int(x) for x in golden["self_grid"])
    cos, sin = tables_fn(ref.wan_freqs(D), grid, D)
    x = torch.from_numpy(golden["self_qhat"]).double().float()
    # rotate the float64 normalised q back and forth through the tables
    ang = golden["self_angles"]
    if not np.allclose(cos.double().numpy(), np.cos(ang), atol=2e-6):
        return False
    if not np.allclose(sin.double().numpy(), np.sin(ang), atol=2e-6):
        return False
    pre = torch.from_numpy(golden["self_q"]).float()
    B, L, H, _ = pre.shape
    g = torch.from_numpy(golden["self_gq"]).float()
    qn = (pre.reshape(B, L, H * D) * torch.rsqrt(pre.reshape(B, L, H * D).pow(2).mean(-1, keepdim=True) + 1e-6) * g)
    got = rope_fn(qn.view(B, L, H, D), cos, sin)
    return float((got.double() - x.double()).abs().max()) < 1e-4


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def test_sdpa_matches_float64_brute_force():
    assert check_attention_vs_brute(lambda q, k, v: ref.sdpa(q, k, v))


def test_brute_force_closed_forms():
    # q = 0 -> uniform weights -> mean of v over the unmasked keys
    k, v = _r((1, 6, 1, D), 3).numpy(), _r((1, 6, 1, D), 4).numpy()
    q = np.zeros((1, 2, 1, D))
    out = ref.brute_attention(q, k, v, seqlen_k=[4])
    assert np.allclose(out[0, :, 0], v[0, :4, 0].mean(0), atol=1e-12)
    # one key far ahead of the rest -> its value
    q = np.zeros((1, 1, 1, D)); q[0, 0, 0, 0] = 1.0
    k = np.zeros((1, 5, 1, D)); k[0, 2, 0, 0] = 1e4
    out = ref.brute_attention(q, k, v[:, :5])
    assert np.allclose(out[0, 0, 0], v[0, 2, 0], atol=1e-12)


def test_sdpa_masking():
    assert check_mask(lambda q, k, v, seqlen_k: ref.sdpa(q, k, v, seqlen_k=seqlen_k))
    q, k, v = _r((1, 5, 2, D), 7), _r((1, 9, 2, D), 8), _r((1, 9, 2, D), 9)
    assert torch.equal(ref.sdpa(q, k, v, seqlen_k=9), ref.sdpa(q, k, v))
    one = ref.sdpa(q, k, v, seqlen_k=1)
    assert torch.allclose(one, v[:, :1].expand(-1, 5, -1, -1), atol=1e-6)
    k2, v2 = k.clone(), v.clone()
    k2[:, 6:] = 1e3
    v2[:, 6:] = -7.0
    assert torch.equal(ref.sdpa(q, k, v, seqlen_k=6), ref.sdpa(q, k2, v2, seqlen_k=6))


def test_sdpa_default_scale_is_inverse_sqrt_d():
    q, k, v = _r((1, 4, 1, D), 1), _r((1, 4, 1, D), 2), _r((1, 4, 1, D), 3)
    want = ref.brute_attention(q.numpy(), k.numpy(), v.numpy(), scale=1 / math.sqrt(D))
    assert np.abs(ref.sdpa(q, k, v).double().numpy() - want).max() < 1e-5


def test_golden_self_path_fp32(golden):
    q, k, v = (torch.from_numpy(golden[f"self_{n}"]) for n in "qkv")
    gq, gk = torch.from_numpy(golden["self_gq"]), torch.from_numpy(golden["self_gk"])
    grid = tuple(int(x) for x in golden["self_grid"])
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    out = ref.self_attn_path(q, k, v, gq, gk, cos, sin)
    assert ref.rel_rms(out, torch.from_numpy(golden["self_out"])) < 1e-5


def test_golden_self_path_bf16(golden):
    """The reference's bf16 rounding points stay within bf16 rounding of the exact answer."""
    q, k, v = (torch.from_numpy(golden[f"self_{n}"]).bfloat16() for n in "qkv")
    gq = torch.from_numpy(golden["self_gq"]).bfloat16()
    gk = torch.from_numpy(golden["self_gk"]).bfloat16()
    grid = tuple(int(x) for x in golden["self_grid"])
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    out = ref.self_attn_path(q, k, v, gq, gk, cos, sin)
    assert ref.rel_rms(out.float(), torch.from_numpy(golden["self_out"])) < 2 ** -6


def test_golden_cross_path(golden):
    q, ck, cv = (torch.from_numpy(golden[f"cross_{n}"]) for n in "qkv")
    gq = torch.from_numpy(golden["cross_gq"])
    out = ref.cross_attn_path(q, ck, cv, gq, seqlen_k=golden["cross_lens"].tolist())
    assert ref.rel_rms(out, torch.from_numpy(golden["cross_out"])) < 1e-5


def test_golden_plain_masked(golden):
    q, k, v = (torch.from_numpy(golden[f"plain_{n}"]) for n in "qkv")
    out = ref.sdpa(q, k, v, seqlen_k=int(golden["plain_len"]))
    assert ref.rel_rms(out, torch.from_numpy(golden["plain_out"])) < 1e-5


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def test_rms_constant_row_closed_form():
    c, C = 0.37, 384
    x = torch.full((1, 3, C), c)
    g = torch.linspace(0.5, 2.0, C)
    want = c / math.sqrt(c * c + 1e-6) * g
    assert torch.allclose(ref.rms(x, g)[0, 1], want, rtol=1e-6)


def test_rms_unit_mean_square_and_scale_invariance():
    x = _r((2, 5, 3072), 11)
    y = ref.rms(x, torch.ones(3072))
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(2, 5), atol=1e-4)
    assert torch.allclose(ref.rms(x * 37.0, torch.ones(3072)), y, atol=1e-5)
    qn, kn = ref.rms_qk(x, 3 * x, torch.ones(3072), torch.ones(3072))
    assert torch.allclose(qn, kn, atol=1e-5)


def test_rms_bf16_rounding_points():
    """bf16 inputs: result equals rounding the fp32 normalised value, then x gamma, in bf16."""
    x = _r((1, 4, 3072), 12).bfloat16()
    g = (1 + torch.rand(3072, generator=torch.Generator().manual_seed(1))).bfloat16()
    y = ref.rms(x, g)
    assert y.dtype == torch.bfloat16
    exact = ref.rms(x.float(), g.float())
    # two roundings of relative size <= 2^-9 each
    assert float(((y.float() - exact).abs() / exact.abs().clamp_min(1e-3)).max()) <= 2 ** -7


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def test_rope_angle_formula_and_split():
    fr = ref.wan_freqs(D)
    assert fr.shape == (1024, 64)
    p = 17
    for lo, dim in ((0, 44), (22, 42), (43, 42)):
        for j in range(dim // 2):
            want = p * 10000.0 ** (-2.0 * j / dim)
            assert abs(float(fr[p, lo + j]) - want) <= 2e-6 * max(1.0, want)


def test_rope_tables_token_order():
    grid = (3, 4, 5)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    ang = torch.atan2(sin, cos)
    fr = ref.wan_freqs(D)
    t, y, x = 2, 3, 1
    tok = t * 20 + y * 5 + x
    want = torch.cat([fr[t, :22], fr[y, 22:43], fr[x, 43:64]])
    assert torch.allclose(torch.cos(ang[tok]), torch.cos(want), atol=1e-6)


def test_rope_identity_at_origin_and_norm_preserved():
    grid = (2, 3, 4)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    x = _r((1, 24, 2, D), 5)
    y = ref.rope(x, cos, sin)
    assert torch.equal(y[:, 0], x[:, 0])
    n_x = x.view(1, 24, 2, 64, 2).pow(2).sum(-1)
    n_y = y.view(1, 24, 2, 64, 2).pow(2).sum(-1)
    assert torch.allclose(n_x, n_y, rtol=1e-5, atol=1e-5)


def test_rope_relative_position():
    """<R(p) q, R(p') k> depends only on p - p' (per axis)."""
    grid = (4, 4, 4)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    q = _r((1, 1, 1, D), 21).expand(1, 64, 1, D).contiguous()
    k = _r((1, 1, 1, D), 22).expand(1, 64, 1, D).contiguous()
    rq, rk = ref.rope(q.double(), cos.double(), sin.double()), ref.rope(k.double(), cos.double(), sin.double())

    def idx(t, y, x):
        return t * 16 + y * 4 + x
    a = float((rq[0, idx(2, 1, 3), 0] * rk[0, idx(1, 0, 2), 0]).sum())
    b = float((rq[0, idx(3, 2, 1), 0] * rk[0, idx(2, 1, 0), 0]).sum())
    assert abs(a - b) < 1e-5 * max(1.0, abs(a))


def test_rope_matches_expanded_table_kernel_form():
    grid = (2, 3, 5)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    x = _r((1, 30, 3, D), 31)
    got = ref.rope(x.double(), cos.double(), sin.double())[0].numpy()
    want = ref.rope_expanded(x[0].double().numpy(), cos.double().numpy(), sin.double().numpy())
    assert np.abs(got - want).max() < 1e-12


def test_rope_golden(golden):
    assert check_rope_golden(ref.rope, ref.rope_tables, golden)


# ---------------------------------------------------------------------------
# planted mistakes: each mutant of the oracle fails at least one of the checks
# ---------------------------------------------------------------------------

def _sdpa_no_scale(q, k, v, seqlen_k=None):
    return ref.sdpa(q, k, v, scale=1.0, seqlen_k=seqlen_k)


def _sdpa_k_channels_reversed(q, k, v, seqlen_k=None):
    # a K operand read with the wrong channel order
    return ref.sdpa(q, k.flip(-1), v, seqlen_k=seqlen_k)


def _sdpa_v_for_k(q, k, v, seqlen_k=None):
    # the two operands swapped
    return ref.sdpa(q, v, k, seqlen_k=seqlen_k)


def _sdpa_mask_off_by_one(q, k, v, seqlen_k=None):
    lens = [x + 1 if x < k.shape[1] else x for x in seqlen_k] if seqlen_k is not None else None
    return ref.sdpa(q, k, v, seqlen_k=lens)


def _sdpa_no_mask(q, k, v, seqlen_k=None):
    return ref.sdpa(q, k, v)


def _rope_wrong_sign(x, cos, sin):
    return ref.rope(x, cos, -sin)


def _rope_swapped_halves(x, cos, sin):
    B, L, n, d = x.shape
    xp = x.float().reshape(B, L, n, 2, d // 2)  # pairs (j, j + d/2) instead of (2j, 2j+1)
    c, s = cos.view(1, L, 1, -1), sin.view(1, L, 1, -1)
    xr, xi = xp[..., 0, :], xp[..., 1, :]
    return torch.stack([xr * c - xi * s, xr * s + xi * c], dim=-2).reshape(B, L, n, d).to(x.dtype)


def _tables_wrong_split(freqs, grid, head_dim):
    f, h, w = grid
    c = head_dim // 2
    fr = freqs.float().split([c // 3, c // 3, c - 2 * (c // 3)], dim=1)  # 21/21/22 instead of 22/21/21
    ang = torch.cat([fr[0][:f].view(f, 1, 1, -1).expand(f, h, w, -1),
                     fr[1][:h].view(1, h, 1, -1).expand(f, h, w, -1),
                     fr[2][:w].view(1, 1, w, -1).expand(f, h, w, -1)], dim=-1).reshape(f * h * w, c)
    return torch.cos(ang), torch.sin(ang)


def _tables_swapped_hw(freqs, grid, head_dim):
    f, h, w = grid
    c, s = ref.rope_tables(freqs, (f, w, h), head_dim)
    return c.view(f, w, h, -1).transpose(1, 2).reshape(f * h * w, -1), s.view(f, w, h, -1).transpose(1, 2).reshape(f * h * w, -1)


@pytest.mark.parametrize("mutant", [_sdpa_no_scale, _sdpa_k_channels_reversed, _sdpa_v_for_k])
def test_planted_attention_mistakes_are_caught(mutant):
    assert not check_attention_vs_brute(lambda q, k, v: mutant(q, k, v))


@pytest.mark.parametrize("mutant", [_sdpa_mask_off_by_one, _sdpa_no_mask])
def test_planted_mask_mistakes_are_caught(mutant):
    assert not check_mask(mutant)


@pytest.mark.parametrize("rope_fn,tables_fn", [
    (_rope_wrong_sign, ref.rope_tables),
    (_rope_swapped_halves, ref.rope_tables),
    (ref.rope, _tables_wrong_split),
    (ref.rope, _tables_swapped_hw),
])
def test_planted_rope_mistakes_are_caught(rope_fn, tables_fn, golden):
    assert not check_rope_golden(rope_fn, tables_fn, golden)


def test_planted_rms_mistakes_are_caught(golden):
    q, k, v = (torch.from_numpy(golden[f"self_{n}"]) for n in "qkv")
    gq, gk = torch.from_numpy(golden["self_gq"]), torch.from_numpy(golden["self_gk"])
    grid = tuple(int(x) for x in golden["self_grid"])
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    want = torch.from_numpy(golden["self_out"])
    B, L, H, _ = q.shape

    def path(normfn):
        qn = normfn(q.reshape(B, L, H * D), gq).view(B, L, H, D)
        kn = normfn(k.reshape(B, L, H * D), gk).view(B, L, H, D)
        return ref.sdpa(ref.rope(qn, cos, sin), ref.rope(kn, cos, sin), v)

    per_head = lambda x, g: (x.view(B, L, H, D) * torch.rsqrt(x.view(B, L, H, D).pow(2).mean(-1, keepdim=True) + 1e-6)).reshape(B, L, H * D) * g  # noqa: E731
    no_gamma = lambda x, g: ref.rms(x, torch.ones_like(g))  # noqa: E731
    assert ref.rel_rms(path(ref.rms), want) < 1e-5
    assert ref.rel_rms(path(per_head), want) > 1e-3
    assert ref.rel_rms(path(no_gamma), want) > 1e-3


# ---------------------------------------------------------------------------
# adaLN stage (ref.adaln): LayerNorm against float64, closed forms of the
# modulation / gate, the per-frame row mapping, and planted mistakes
# ---------------------------------------------------------------------------

def _bf16_ulp_close(got: torch.Tensor, want64: np.ndarray, ulps: float = 1.0) -> bool:
    """|got - want| within `ulps` bf16 ulps of |want| (absolute floor 2^-30)."""
    g = got.double().numpy()
    w = np.asarray(want64, dtype=np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(w), 2.0 ** -30))) - 7)
    return bool((np.abs(g - w) <= ulps * ulp).all())


def check_adaln_layer_norm(fn) -> bool:
    x = (_r((2, 6, 256), 40) * 3 + 1).bfloat16()
    w, b = (1 + 0.3 * _r((256,), 41)).bfloat16(), (0.2 * _r((256,), 42)).bfloat16()
    _, h = fn(x, ln_weight=w, ln_bias=b)
    want = ref.layer_norm64(x.double().numpy(), w.double().numpy(), b.double().numpy(), ref.EPS)
    _, h0 = fn(x)
    want0 = ref.layer_norm64(x.double().numpy(), eps=ref.EPS)
    return _bf16_ulp_close(h, want) and _bf16_ulp_close(h0, want0)


def check_adaln_frames_and_gate(fn) -> bool:
    """Frame f's tokens take row f of e: with scale = -1 the modulation returns the shift row
    exactly; a zero gate leaves x, a unit gate gives bf16(x + y), no gate adds y."""
    B, Fr, per, C = 2, 3, 5, 64
    x, y = _r((B, Fr * per, C), 43).bfloat16(), _r((B, Fr * per, C), 44).bfloat16()
    e = torch.zeros(Fr, 6, C)
    e[:, 1] = -1.0                                       # scale row: 1 + scale = 0
    e[:, 0] = torch.arange(Fr, dtype=torch.float32).view(Fr, 1) + 0.5 * torch.arange(C) / C
    e[:, 2] = torch.tensor([0.0, 1.0, 0.0]).view(Fr, 1)  # gate row: 0 / 1 / 0 by frame
    e = e.bfloat16()
    _, h = fn(x, e=e, frames=Fr, shift_idx=0, scale_idx=1)
    want_h = e[:, 0].unsqueeze(1).expand(Fr, per, C).reshape(1, Fr * per, C).expand(B, -1, -1)
    r, _ = fn(x, y, e=e, frames=Fr, gate_idx=2, norm=False)
    gmask = torch.tensor([0.0, 1.0, 0.0]).repeat_interleave(per).view(1, -1, 1).bool()
    want_r = torch.where(gmask, (x.float() + y.float()).bfloat16(), x)
    r2, _ = fn(x, y, norm=False)
    return (torch.equal(h, want_h) and torch.equal(r, want_r)
            and torch.equal(r2, (x.float() + y.float()).bfloat16()))


def check_adaln_zero_modulation(fn) -> bool:
    x = _r((1, 8, 128), 45).bfloat16()
    e = torch.zeros(2, 6, 128).bfloat16()
    _, h = fn(x, e=e, frames=2, shift_idx=3, scale_idx=4)
    _, ln = fn(x)
    return torch.equal(h, ln)


def test_adaln_layer_norm_matches_float64():
    assert check_adaln_layer_norm(ref.adaln)


def test_adaln_layer_norm_known_answer():
    x = torch.tensor([[[1.0, 2.0, 3.0, 4.0]]]).bfloat16()
    _, h = ref.adaln(x, eps=0.0)
    want = (np.array([1, 2, 3, 4]) - 2.5) / math.sqrt(1.25)
    assert _bf16_ulp_close(h[0, 0], want)


def test_adaln_frames_gate_and_zero_modulation():
    assert check_adaln_frames_and_gate(ref.adaln)
    assert check_adaln_zero_modulation(ref.adaln)


def _adaln_unbiased_var(x, y=None, e=None, frames=1, gate_idx=-1, shift_idx=-1, scale_idx=-1,
                        ln_weight=None, ln_bias=None, eps=ref.EPS, norm=True):
    r, _ = ref.adaln(x, y, e, frames, gate_idx, norm=False)
    if not norm:
        return r, None
    n = r.shape[-1]
    rf = r.float()
    h = ((rf - rf.mean(-1, keepdim=True)) / torch.sqrt(rf.var(-1, keepdim=True) + eps))
    if ln_weight is not None:
        h = h * ln_weight.float() + ln_bias.float()
    h = h.bfloat16()
    assert n > 1
    if shift_idx >= 0:
        B, L, C = h.shape
        h = (h.view(B, frames, L // frames, C) * (1 + e[:, scale_idx].unsqueeze(0).unsqueeze(2))
             + e[:, shift_idx].unsqueeze(0).unsqueeze(2)).view(B, L, C)
    return r, h


def _adaln_frames_interleaved(x, y=None, e=None, frames=1, gate_idx=-1, shift_idx=-1, scale_idx=-1,
                              ln_weight=None, ln_bias=None, eps=ref.EPS, norm=True):
    # token l taken as frame l % frames instead of l // (L / frames)
    B, L, C = x.shape
    perm = torch.arange(L).view(L // frames, frames).t().reshape(-1)
    inv = torch.argsort(perm)
    r, h = ref.adaln(x[:, perm], None if y is None else y[:, perm], e, frames, gate_idx, shift_idx,
                     scale_idx, ln_weight, ln_bias, eps, norm)
    return r[:, inv], None if h is None else h[:, inv]


def _adaln_gate_on_x(x, y=None, e=None, frames=1, gate_idx=-1, shift_idx=-1, scale_idx=-1,
                     ln_weight=None, ln_bias=None, eps=ref.EPS, norm=True):
    # the gate multiplies the residual instead of the branch output
    if y is not None and gate_idx >= 0:
        B, L, C = x.shape
        xg = (x.view(B, frames, L // frames, C) * e[:, gate_idx].unsqueeze(0).unsqueeze(2)).view(B, L, C)
        return ref.adaln(xg, y, None, frames, -1, shift_idx, scale_idx, ln_weight, ln_bias, eps, norm)
    return ref.adaln(x, y, e, frames, gate_idx, shift_idx, scale_idx, ln_weight, ln_bias, eps, norm)


@pytest.mark.parametrize("mutant", [_adaln_unbiased_var, _adaln_frames_interleaved, _adaln_gate_on_x])
def test_planted_adaln_mistakes_are_caught(mutant):
    ok = (check_adaln_layer_norm(mutant) and check_adaln_frames_and_gate(mutant)
          and check_adaln_zero_modulation(mutant))
    assert not ok
