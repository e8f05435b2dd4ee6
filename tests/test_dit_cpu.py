"""Host logic of the block / DiT mirror (fast_dit.py) and the oracle's block and DiT
forward, on the CPU with a tiny model (head_dim 128, 2 heads, 2 layers).

  * oracle.block_forward: identity when every branch output is zero; only the cross
    branch survives when the adaLN gates are zero (residual and gate wiring);
  * oracle.unpatchify: the explicit index map of einsum 'fhwpqrc->cfphqwr';
  * oracle.block_forward modulation rows: scale = -1 turns a LayerNorm stage into its shift
    row, which makes the self branch lin_o(lin_v(s)) and the FFN branch ffn(s) in closed
    form (planted shift/scale swaps fail); gates per frame;
  * the FFN and the text embedding use the tanh form of GELU (a planted erf form fails);
  * FastWanDiT with FAST_ATTN_IMPL="sdpa" (bf16 weights) against oracle.dit_forward
    (fp32 copy of the same weights): the whole CFG noise prediction.
The HIP ("hip") backend of the same code runs in tests/test_gpu_dit.py.
"""
import copy
import math

import torch

from oracle import ref

TINY = dict(dim=256, ffn_dim=512, num_heads=2, num_layers=2, in_dim=4, out_dim=4, text_dim=64,
            freq_dim=32)


def _tiny(W, dtype=torch.bfloat16, seed=0):
    cfg = W.model.WanConfig(**TINY)
    return W.model.random_model(cfg, device="cpu", dtype=dtype, std=0.05, seed=seed)


def test_block_forward_residual_and_gate_wiring(W):
    m = _tiny(W, torch.float32)
    blk = copy.deepcopy(m.blocks[0])
    B, grid = 2, (2, 3, 4)
    L = 24
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, L, 256, generator=g)
    e0 = torch.randn(1, 2, 6, 256, generator=g) * 0.1
    cos, sin = ref.rope_tables(ref.wan_freqs(128), grid, 128)
    ck, cv = torch.randn(B, 5, 2, 128, generator=g), torch.randn(B, 5, 2, 128, generator=g)
    with torch.no_grad():
        for lin in (blk.self_attn.o, blk.cross_attn.o, blk.ffn[2]):
            lin.weight.zero_()
            lin.bias.zero_()
    assert torch.allclose(ref.block_forward(blk, x, e0, cos, sin, ck, cv, 2), x, atol=1e-6)
    blk2 = copy.deepcopy(m.blocks[0])
    e0g = e0.clone()
    e0g[:, :, 2] = -blk2.modulation[0, 2].detach()
    e0g[:, :, 5] = -blk2.modulation[0, 5].detach()
    out = ref.block_forward(blk2, x, e0g, cos, sin, ck, cv, 2)
    ca = blk2.cross_attn
    h = torch.nn.functional.layer_norm(x, (256,), blk2.norm3.weight, blk2.norm3.bias, eps=1e-6)
    q = ref._rms32(ref._lin32(h, ca.q), ca.norm_q).view(B, L, 2, 128)
    cross = ref._lin32(ref.sdpa(q, ck, cv).reshape(B, L, 256), ca.o)
    assert torch.allclose(out, x + cross, atol=1e-5)


def test_unpatchify_index_map():
    grid, patch, c = (2, 3, 4), (1, 2, 2), 3
    f, h, w = grid
    y = torch.arange(2 * f * h * w * 4 * c, dtype=torch.float32).view(2, f * h * w, 4 * c)
    out = ref.unpatchify(y, grid, patch, c)
    yv = y.view(2, f, h, w, 1, 2, 2, c)
    for b in range(2):
        for ci in range(c):
            for t in range(f):
                for yy in range(2 * h):
                    for xx in range(2 * w):
                        assert out[b, ci, t, yy, xx] == yv[b, t, yy // 2, xx // 2, 0, yy % 2, xx % 2, ci]


def test_fast_dit_sdpa_matches_fp32_oracle(W):
    m = _tiny(W)
    grid = (3, 4, 5)
    fast = W.fast_dit.FastWanDiT(m, grid, guide_scale=5.0, attn_impl="sdpa", cross_impl="sdpa")
    g = torch.Generator().manual_seed(2)
    latent = torch.randn(4, 3, 8, 10, generator=g)
    ctx_c, ctx_n = torch.randn(1, 7, 64, generator=g), torch.randn(1, 7, 64, generator=g)
    fast.set_context(ctx_c, ctx_n)
    got = fast(latent, torch.tensor(700))
    m32 = copy.deepcopy(m).float()
    want = ref.dit_forward(m32, latent, 700, ctx_c, ctx_n, grid, 5.0)
    assert got.shape == want.shape == (4, 3, 8, 10)
    e = ref.rel_rms(got.float(), want)
    assert e < 3e-2, e


# ─── closed forms of the block's modulation rows and of the GELU form ──────────────
#
# With the scale row of a LayerNorm stage at -1, that stage's output is its shift row for
# every token, whatever x is: h = LN(x) * (1 + (-1)) + shift.  With h the same row s for
# every token, self-attention returns lin_v(s) for every query (all values are equal and
# the softmax weights sum to 1), and the FFN returns ffn(s): the block's output is then a
# closed form of s.  A swap of the shift and scale rows, or an erf-GELU in place of the
# tanh form (wan/modules/model.py:214,379 build nn.GELU(approximate='tanh')), breaks it.

def _gelu_tanh64(x):
    """GELU, tanh approximation (Hendrycks & Gimpel), float64."""
    x = x.double()
    return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def _lin64(x, m):
    return x.double() @ m.weight.double().t() + m.bias.double()


def _zero(*lins):
    with torch.no_grad():
        for lin in lins:
            lin.weight.zero_()
            lin.bias.zero_()


def _block_case(W, seed):
    m = _tiny(W, torch.float32, seed=seed)
    blk = copy.deepcopy(m.blocks[0])
    B, grid, F_ = 2, (2, 3, 4), 2
    L, C = 24, 256
    g = torch.Generator().manual_seed(10 + seed)
    x = torch.randn(B, L, C, generator=g)
    cos, sin = ref.rope_tables(ref.wan_freqs(128), grid, 128)
    ck, cv = torch.randn(B, 5, 2, 128, generator=g), torch.randn(B, 5, 2, 128, generator=g)
    e0 = torch.randn(1, F_, 6, C, generator=g) * 0.3
    return blk, x, e0, cos, sin, ck, cv, g


def _rows(blk, e0):
    """The block's effective modulation rows [F, 6, C] (block modulation + time projection)."""
    return (blk.modulation.detach() + e0[0]).double()


def _set_row(blk, e0, i, value):
    """e0 such that effective row i equals `value` ([C] or [F, C]) in every frame."""
    e0 = e0.clone()
    e0[0, :, i] = value - blk.modulation.detach()[0, i]
    return e0


def _swap_rows(blk, e0, i, j):
    """The same block with modulation rows i and j exchanged (in the block parameter and
    in e0): running the oracle on it is running an oracle that reads e[i] where it should
    read e[j] and vice versa."""
    b2 = copy.deepcopy(blk)
    perm = list(range(6))
    perm[i], perm[j] = j, i
    with torch.no_grad():
        b2.modulation.copy_(blk.modulation[:, perm])
    return b2, e0[:, :, perm].clone()


def _self_branch_closed_form(blk, x, e0, s):
    """x + lin_o(lin_v(s)) * e2 per frame, float64 (cross and FFN branches zeroed)."""
    sa = blk.self_attn
    y = _lin64(_lin64(s[None], sa.v), sa.o)[0]                     # [C]
    e2 = _rows(blk, e0)[:, 2]                                      # [F, C]
    B, L, C = x.shape
    Fr = e2.shape[0]
    return (x.double().view(B, Fr, L // Fr, C) + (y * e2)[None, :, None]).view(B, L, C)


def _ffn_closed_form(blk, x, e0, s, gelu=_gelu_tanh64):
    """x + ffn(s) * e5 per frame, float64 (self and cross branches zeroed)."""
    ffn = blk.ffn
    y = _lin64(gelu(_lin64(s[None], ffn[0])), ffn[2])[0]
    e5 = _rows(blk, e0)[:, 5]
    B, L, C = x.shape
    Fr = e5.shape[0]
    return (x.double().view(B, Fr, L // Fr, C) + (y * e5)[None, :, None]).view(B, L, C)


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def test_block_self_stage_shift_scale_rows_closed_form(W):
    blk, x, e0, cos, sin, ck, cv, g = _block_case(W, 0)
    _zero(blk.cross_attn.o, blk.ffn[2])
    s = torch.randn(256, generator=g)
    e0 = _set_row(blk, _set_row(blk, e0, 1, -1.0), 0, s)
    want = _self_branch_closed_form(blk, x, e0, s.double())
    out = ref.block_forward(blk, x, e0, cos, sin, ck, cv, 2)
    assert _rel(out - x, want - x) < 1e-5
    # planted: shift and scale rows read the other way round
    b2, e2 = _swap_rows(blk, e0, 0, 1)
    bad = ref.block_forward(b2, x, e2, cos, sin, ck, cv, 2)
    assert _rel(bad - x, want - x) > 1e-2


def test_block_ffn_stage_shift_scale_rows_and_gelu_closed_form(W, monkeypatch):
    blk, x, e0, cos, sin, ck, cv, g = _block_case(W, 1)
    _zero(blk.self_attn.o, blk.cross_attn.o)
    s = 4 * torch.randn(256, generator=g)        # pre-activations of a few units: GELU's curved part
    e0 = _set_row(blk, _set_row(blk, e0, 4, -1.0), 3, s)
    want = _ffn_closed_form(blk, x, e0, s.double())
    out = ref.block_forward(blk, x, e0, cos, sin, ck, cv, 2)
    err = _rel(out - x, want - x)
    assert err < 1e-5, err
    # the erf form of GELU is a different closed form, far beyond the fp32 error above
    erf = _ffn_closed_form(blk, x, e0, s.double(), gelu=lambda t: torch.nn.functional.gelu(t))
    assert _rel(erf - x, want - x) > 20 * max(err, 1e-7)
    # planted: shift and scale rows swapped
    b2, e2 = _swap_rows(blk, e0, 3, 4)
    assert _rel(ref.block_forward(b2, x, e2, cos, sin, ck, cv, 2) - x, want - x) > 1e-2
    # planted: the oracle's GELU in the erf form
    real_gelu = torch.nn.functional.gelu
    monkeypatch.setattr(ref.F, "gelu", lambda t, approximate="none": real_gelu(t))
    bad = ref.block_forward(blk, x, e0, cos, sin, ck, cv, 2)
    assert _rel(bad - x, want - x) > 20 * max(err, 1e-7)


def test_block_gate_rows_per_frame(W):
    """Gates e2 / e5 scale their branch per frame: zero in frame 0 and one in frame 1 keep
    x in frame 0 and add the whole branch in frame 1 (a swapped frame map fails)."""
    blk, x, e0, cos, sin, ck, cv, g = _block_case(W, 2)
    _zero(blk.cross_attn.o)
    gate = torch.stack([torch.zeros(256), torch.ones(256)])        # [F, C]
    e0 = _set_row(blk, _set_row(blk, e0, 2, gate), 5, gate)
    out = ref.block_forward(blk, x, e0, cos, sin, ck, cv, 2)
    B, L, C = x.shape
    assert torch.equal(out[:, :L // 2], x[:, :L // 2])
    assert (out[:, L // 2:] - x[:, L // 2:]).abs().max() > 1e-3


def test_text_embedding_is_tanh_gelu(W, monkeypatch):
    m = _tiny(W, torch.float32, seed=3)
    g = torch.Generator().manual_seed(4)
    ctx = 5 * torch.randn(2, 7, 64, generator=g)           # pre-activations spread over GELU's bend
    tx = m.text_embedding
    want = _lin64(_gelu_tanh64(_lin64(ctx, tx[0])), tx[2])
    got = ref.text_context(tx, ctx)
    err = _rel(got, want)
    assert err < 1e-5, err
    erf = _lin64(torch.nn.functional.gelu(_lin64(ctx, tx[0])), tx[2])
    assert _rel(erf, want) > 20 * max(err, 1e-7)
    real_gelu = torch.nn.functional.gelu
    monkeypatch.setattr(ref.F, "gelu", lambda t, approximate="none": real_gelu(t))
    assert _rel(ref.text_context(tx, ctx), want) > 20 * max(err, 1e-7)


def test_qkv_weights_are_packed_once_as_views(W):
    """The fused q/k/v projection's [3C, C] weight holds the only copy: the q, k and v
    parameters become views of it with unchanged values, and a second block wrapper over
    the same module reuses the packed tensors."""
    m = _tiny(W)
    sa = m.blocks[0].self_attn
    before = [t.detach().clone() for t in (sa.q.weight, sa.k.weight, sa.v.weight, sa.q.bias, sa.v.bias)]
    fb = W.fast_dit._FastBlock(m.blocks[0], 2, attn_impl="hip")
    C = sa.q.weight.shape[0]
    assert fb.w_qkv.shape == (3 * C, sa.q.weight.shape[1])
    for i, lin in enumerate((sa.q, sa.k, sa.v)):
        assert lin.weight.data_ptr() == fb.w_qkv[i * C].data_ptr()
        assert lin.bias.data_ptr() == fb.b_qkv[i * C:].data_ptr()
    after = (sa.q.weight, sa.k.weight, sa.v.weight, sa.q.bias, sa.v.bias)
    assert all(torch.equal(a, b) for a, b in zip(before, after))
    fb2 = W.fast_dit._FastBlock(m.blocks[0], 2, attn_impl="hip")
    assert fb2.w_qkv.data_ptr() == fb.w_qkv.data_ptr()
    # a state dict still loads into the views (in place, so the packed copy follows)
    sd = {k: v.clone() + 1 for k, v in m.blocks[0].state_dict().items()}
    m.blocks[0].load_state_dict(sd)
    assert torch.equal(fb.w_qkv[C:2 * C], sd["self_attn.k.weight"])


def test_chained_block_boundaries_equal_separate_stages(W):
    """FastWanDiT does each block boundary in one pointwise call (block i's gated residual
    with block i+1's norm1 + modulation; the last block's with the head's): with the eager
    torch stages the guided prediction equals, bit for bit, running every block's four
    stages and the head's own stage separately."""
    m = _tiny(W)
    grid = (3, 4, 5)
    fast = W.fast_dit.FastWanDiT(m, grid, guide_scale=5.0, attn_impl="sdpa", cross_impl="sdpa",
                                 pointwise_impl="eager")
    g = torch.Generator().manual_seed(3)
    latent = torch.randn(4, 3, 8, 10, generator=g)
    ctx_c, ctx_n = torch.randn(1, 7, 64, generator=g), torch.randn(1, 7, 64, generator=g)
    fast.set_context(ctx_c, ctx_n)
    t = torch.tensor(600)
    got = fast(latent, t)
    e, e0 = fast.time_rows(t)
    x = fast.patch(latent)
    for blk, (ck, cv) in zip(fast.blocks, fast.context):
        x = blk(x, e0, fast.cos, fast.sin, ck, cv, fast.seqlen_k)
    want = W.fast_dit.noise_prediction(m.head, x, e, grid, m.patch_size, m.out_dim, 5.0)
    assert torch.equal(got, want)
