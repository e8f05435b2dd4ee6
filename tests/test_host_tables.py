"""Host-side tables and the oracle's small helpers, pinned on the CPU.

  * the product's RoPE tables (wan2-ti2v-5b_amd/rope.py: wan_freqs, rope_tables) are
    bit-identical to the oracle's and match the float64 angle grid of
    tests/golden/make_golden.py (an independent numpy restatement) at the DiT's grids,
    including (21, 22, 17), the grid of the reference's block bench
    (scripts/validate/block_bench.py:34), and the golden rotation fixture;
  * sinusoidal_embedding_1d (wan/modules/model.py:15-25), product and oracle, against its
    closed form: position 0 is [1 ... 1 | 0 ... 0], known values at dim 4;
  * oracle.inv_rms: a constant row's closed form, and x * inv * gamma == oracle.rms(x, gamma)
    in fp32;
  * the CFG combine uncond + g (cond - uncond) (models/fast_dit.py:504-505) in both the
    oracle's dit_forward and the product's FastWanDiT: g = 1 returns the cond prediction,
    g = 0 the uncond one, each anchored by a run whose two contexts are equal (where the
    prediction cannot depend on g), and a planted swap of cond and uncond fails the check.
"""
import copy
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import ref

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402  (float64 numpy angle grid, independent of the oracle)

from test_oracle import check_rope_golden  # noqa: E402

D = 128
GRIDS = [(21, 17, 22), (21, 22, 17), (6, 12, 15), (3, 4, 5), (1, 1, 1)]


# ---------------------------------------------------------------------------
# RoPE tables of the product
# ---------------------------------------------------------------------------

def test_product_freqs_equal_oracle_and_closed_form(W):
    fr = W.rope.wan_freqs(D)
    assert torch.equal(fr, ref.wan_freqs(D))
    assert fr.shape == (1024, 64) and fr.dtype == torch.float32
    for p in (0, 1, 20, 1023):
        for lo, dim in ((0, 44), (22, 42), (43, 42)):
            for j in range(dim // 2):
                want = p * 10000.0 ** (-2.0 * j / dim)
                assert abs(float(fr[p, lo + j]) - want) <= 2e-6 * max(1.0, want)


@pytest.mark.parametrize("grid", GRIDS)
def test_product_rope_tables_equal_oracle(W, grid):
    cos, sin = W.rope.rope_tables(W.rope.wan_freqs(D), grid, D)
    rc, rs = ref.rope_tables(ref.wan_freqs(D), grid, D)
    L = grid[0] * grid[1] * grid[2]
    assert cos.shape == sin.shape == (L, 64) and cos.is_contiguous() and sin.is_contiguous()
    assert torch.equal(cos, rc) and torch.equal(sin, rs)


@pytest.mark.parametrize("grid", [(21, 17, 22), (21, 22, 17), (6, 12, 15)])
def test_product_rope_tables_vs_float64_angles(W, grid):
    """cos/sin against np.cos / np.sin of the float64 angle grid: the fp32 angle of position
    p <= 21 is within ~2e-6 of the exact one, so the tables are too."""
    cos, sin = W.rope.rope_tables(W.rope.wan_freqs(D), grid, D)
    ang = make_golden.angles(grid)
    assert np.abs(cos.double().numpy() - np.cos(ang)).max() < 4e-6
    assert np.abs(sin.double().numpy() - np.sin(ang)).max() < 4e-6
    if grid[1] != grid[2]:
        # the two grids of L=7854 differ: height and width are not interchangeable
        swapped = make_golden.angles((grid[0], grid[2], grid[1]))
        assert np.abs(cos.double().numpy() - np.cos(swapped)).max() > 1e-2


def test_product_rope_tables_golden_rotation(W, golden):
    def tables(freqs, grid, d):
        return W.rope.rope_tables(W.rope.wan_freqs(d), grid, d)
    assert check_rope_golden(W.fast_dit._rope, tables, golden)


def test_model_freqs_are_the_product_tables(W):
    cfg = W.model.WanConfig(dim=256, ffn_dim=512, num_heads=2, num_layers=1, in_dim=4, out_dim=4,
                            text_dim=64, freq_dim=32)
    m = W.model.random_model(cfg, device="cpu", seed=0)
    assert torch.equal(m.freqs, ref.wan_freqs(D))


# ---------------------------------------------------------------------------
# sinusoidal time embedding
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("which", ["product", "oracle"])
def test_sinusoidal_embedding_closed_form(W, which):
    fn = W.model.sinusoidal_embedding_1d if which == "product" else ref.sinusoidal_embedding_1d
    e0 = fn(256, torch.tensor([0.0]))
    assert e0.dtype == torch.float64 and e0.shape == (1, 256)
    assert torch.equal(e0[0, :128], torch.ones(128, dtype=torch.float64))
    assert torch.equal(e0[0, 128:], torch.zeros(128, dtype=torch.float64))
    e1 = fn(4, torch.tensor([1.0]))[0].tolist()
    want = [math.cos(1.0), math.cos(0.01), math.sin(1.0), math.sin(0.01)]
    assert np.allclose(e1, want, rtol=0, atol=1e-15)
    pos = torch.tensor([0.0, 3.0, 500.0, 999.0])
    got = fn(256, pos).numpy()
    freq = 10000.0 ** (-np.arange(128) / 128.0)
    arg = np.outer(pos.numpy(), freq)
    assert np.allclose(got, np.concatenate([np.cos(arg), np.sin(arg)], 1), rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# oracle.inv_rms
# ---------------------------------------------------------------------------

def test_inv_rms_closed_form_and_rms_identity():
    c, eps = 0.75, 1e-6
    x = torch.full((2, 3, 384), c)
    inv = ref.inv_rms(x, eps)
    assert inv.shape == (2, 3)
    assert torch.allclose(inv, torch.full((2, 3), 1.0 / math.sqrt(c * c + eps)), rtol=1e-6)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 17, 384, generator=g) * 2.5
    gamma = 1 + torch.rand(384, generator=g)
    inv = ref.inv_rms(x, eps)
    assert torch.allclose(x * inv.unsqueeze(-1) * gamma, ref.rms(x, gamma, eps), rtol=1e-6, atol=1e-6)
    # independent float64 statistic
    x64 = x.double().numpy()
    want = 1.0 / np.sqrt((x64 ** 2).mean(-1) + eps)
    assert np.allclose(inv.double().numpy(), want, rtol=2e-6)


# ---------------------------------------------------------------------------
# CFG combine
# ---------------------------------------------------------------------------

TINY = dict(dim=256, ffn_dim=512, num_heads=2, num_layers=1, in_dim=4, out_dim=4, text_dim=64,
            freq_dim=32)


def _tiny_inputs():
    g = torch.Generator().manual_seed(12)
    latent = torch.randn(4, 2, 6, 8, generator=g)
    ctx_c, ctx_n = torch.randn(1, 5, 64, generator=g), torch.randn(1, 5, 64, generator=g)
    return latent, ctx_c, ctx_n


def _check_cfg(pred, tol):
    """pred(g, ctx_first, ctx_second) -> noise prediction with [ctx_first, ctx_second] as
    [cond, uncond].  With both contexts equal the prediction is that context's own (any g):
    g = 1 must return the cond one, g = 0 the uncond one, and g = 5 the affine combination."""
    _, c, n = _tiny_inputs()
    yc, yn = pred(1.0, c, c), pred(1.0, n, n)
    close = lambda a, b, t=tol: ref.rel_rms(a, b) < t   # noqa: E731
    if close(yc, yn, 20 * tol):      # the two contexts must give clearly different predictions
        return False
    return (close(pred(1.0, c, n), yc) and close(pred(0.0, c, n), yn)
            and close(pred(5.0, c, n), yn + 5.0 * (yc - yn), 5 * tol))


def _oracle_pred(m32, swap=False):
    latent, _, _ = _tiny_inputs()

    def pred(gs, a, b):
        # planted mistake when swap: cond + g (uncond - cond), i.e. the two exchanged
        return ref.dit_forward(m32, latent, 600, a, b, (2, 3, 4), 1.0 - gs if swap else gs)
    return pred


def test_oracle_cfg_combine(W):
    cfg = W.model.WanConfig(**TINY)
    m32 = W.model.random_model(cfg, device="cpu", dtype=torch.float32, std=0.05, seed=4)
    assert _check_cfg(_oracle_pred(m32), 1e-5)
    assert not _check_cfg(_oracle_pred(m32, swap=True), 1e-5)


def test_product_cfg_combine(W):
    """The product's head (bf16, as FastWanDiT runs it) on the CPU with the sdpa backend."""
    cfg = W.model.WanConfig(**TINY)
    m = W.model.random_model(cfg, device="cpu", std=0.05, seed=4)
    latent, c, n = _tiny_inputs()

    def pred(gs, a, b):
        fast = W.fast_dit.FastWanDiT(m, (2, 3, 4), gs, attn_impl="sdpa", cross_impl="sdpa",
                                     pointwise_impl="eager")
        fast.set_context(a, b)
        return fast(latent, torch.tensor(600)).float()
    assert _check_cfg(pred, 1e-2)
    # and it agrees with the oracle's fp32 forward of the same weights
    want = ref.dit_forward(copy.deepcopy(m).float(), latent, 600, c, n, (2, 3, 4), 5.0)
    assert ref.rel_rms(pred(5.0, c, n), want) < 3e-2
