"""GPU: the fused adaLN stages (ops.adaln, wan_adaln) against the CPU oracle (ref.adaln).

The residual update r is exact elementwise bf16 arithmetic and must match bit for bit.
The normalised / modulated row h follows the same bf16 rounding points as the oracle;
the only difference allowed is the order of the fp32 LayerNorm sums, which can move a
value across a bf16 rounding boundary: at most 2 bf16 ulps (at magnitude >= 1) on at
most 1% of the elements.
"""
import numpy as np
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# (gate_idx, shift_idx, scale_idx, affine, with_y, norm): the four stages of a block
STAGES = {
    "norm1_modulate": (-1, 0, 1, False, False, True),     # models/fast_dit.py:280
    "gate_residual_norm3": (2, -1, -1, True, True, True),  # :294 then norm3
    "residual_norm2_modulate": (-1, 3, 4, False, True, True),  # :306-307
    "gate_residual": (5, -1, -1, False, True, False),      # :311
}


def _inputs(B, L, C, Fr, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, L, C, generator=g) * 2 + 0.5).bfloat16()
    y = torch.randn(B, L, C, generator=g).bfloat16()
    e = (torch.randn(Fr, 6, C, generator=g) * 0.5).bfloat16()
    w = (1 + 0.2 * torch.randn(C, generator=g)).bfloat16()
    b = (0.1 * torch.randn(C, generator=g)).bfloat16()
    return x, y, e, w, b


def _compare_h(got, want):
    g, w = got.double(), want.double()
    diff = (g - w).abs()
    tol = 2 * torch.exp2(torch.floor(torch.log2(w.abs().clamp_min(1.0))) - 7)
    bad = diff > tol
    frac = float((diff > 0).double().mean())
    return int(bad.sum()), frac


def _run(W, stage, B, L, C, Fr, seed):
    gate, shift, scale, affine, with_y, norm = STAGES[stage]
    x, y, e, w, b = _inputs(B, L, C, Fr, seed)
    kw = dict(e=e, frames=Fr, gate_idx=gate, shift_idx=shift, scale_idx=scale,
              ln_weight=w if affine else None, ln_bias=b if affine else None, eps=1e-6, norm=norm)
    r_want, h_want = ref.adaln(x, y if with_y else None, **kw)
    kwd = dict(kw, e=e.to(DEV), ln_weight=w.to(DEV) if affine else None,
               ln_bias=b.to(DEV) if affine else None)
    r, h = W.ops.adaln(x.to(DEV), y.to(DEV) if with_y else None, **kwd)
    torch.cuda.synchronize()
    assert torch.equal(r.cpu(), r_want), f"{stage}: residual differs"
    if norm:
        nbad, frac = _compare_h(h.cpu(), h_want)
        print(f"{stage} B={B} L={L} C={C} F={Fr}: h differs on {frac:.2e} of elements")
        assert nbad == 0 and frac <= 1e-2
    else:
        assert h is None


@pytest.mark.parametrize("stage", list(STAGES))
def test_block_stages(W, stage):
    _run(W, stage, 2, 60, 3072, 3, 1)


@pytest.mark.parametrize("C", [256, 1000, 2048, 4096, 8192])
def test_dims(W, C):
    """Every lanes-per-row template, including a partial last chunk (C=1000)."""
    _run(W, "gate_residual_norm3", 1, 12, C, 4, C)
    _run(W, "residual_norm2_modulate", 1, 12, C, 4, C + 1)


def test_full_size_stage(W):
    """norm1 + modulate at the block's real shape: B=2, L=7854 (21 frames), C=3072."""
    _run(W, "norm1_modulate", 2, 7854, 3072, 21, 7)


def test_outputs_are_layer_norm_statistics(W):
    """Size-independent check at full size: without affine or modulation, every row of h
    has mean ~0 and mean square ~1 (within bf16 rounding)."""
    x, _, _, _, _ = _inputs(2, 7854, 3072, 21, 9)
    _, h = W.ops.adaln(x.to(DEV))
    hf = h.float()
    assert float(hf.mean(-1).abs().max()) < 2e-3
    assert float((hf.pow(2).mean(-1) - 1).abs().max()) < 1e-2


@pytest.mark.parametrize("mod_rows,shift,scale", [(6, 0, 1), (2, 0, 1)])
def test_boundary_stage_equals_two_stages(W, mod_rows, shift, scale):
    """wan_adaln_ex: one block's gated residual (gate e[5]) and the following stage's
    LayerNorm + modulation from another row set in one pass, at B=2, L=7854, 21 frames: the
    next block's norm1 + modulate (6 rows per frame) and the output head's (2 rows).  Both
    outputs must equal the two separate stages bit for bit (the residual is rounded to bf16
    before its statistics, exactly as when the second stage re-reads it); h also against the
    oracle's rounding points."""
    B, L, C, Fr = 2, 7854, 3072, 21
    x, y, e, _, _ = _inputs(B, L, C, Fr, 21)
    g = torch.Generator().manual_seed(22)
    e_mod = (torch.randn(Fr, mod_rows, C, generator=g) * 0.5).bfloat16()
    xd, yd, ed, md = (t.to(DEV) for t in (x, y, e, e_mod))
    r1, _ = W.ops.adaln(xd, yd, ed, Fr, gate_idx=5, norm=False)
    e6 = md if mod_rows == 6 else torch.zeros(Fr, 6, C, dtype=torch.bfloat16, device=DEV)
    if mod_rows != 6:
        e6[:, :mod_rows] = md
    _, h1 = W.ops.adaln(r1, None, e6.contiguous(), Fr, shift_idx=shift, scale_idx=scale)
    r2, h2 = W.ops.adaln(xd, yd, ed, Fr, gate_idx=5, shift_idx=shift, scale_idx=scale, e_mod=md)
    torch.cuda.synchronize()
    assert torch.equal(r2, r1) and torch.equal(h2, h1)
    # the oracle: gate + residual, then LayerNorm + modulation with the other rows
    r_want, _ = ref.adaln(x, y, e, Fr, gate_idx=5, norm=False)
    _, h_want = ref.adaln(r_want, None, e6.cpu(), Fr, shift_idx=shift, scale_idx=scale)
    assert torch.equal(r2.cpu(), r_want)
    nbad, frac = _compare_h(h2.cpu(), h_want)
    print(f"boundary stage, {mod_rows} modulation rows: bit-identical to two stages; "
          f"h differs from the oracle on {frac:.2e} of elements")
    assert nbad == 0 and frac <= 1e-2
