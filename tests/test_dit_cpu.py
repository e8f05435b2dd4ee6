"""Host logic of the block / DiT mirror (fast_dit.py) and the oracle's block and DiT
forward, on the CPU with a tiny model (head_dim 128, 2 heads, 2 layers).

  * oracle.block_forward: identity when every branch output is zero; only the cross
    branch survives when the adaLN gates are zero (residual and gate wiring);
  * oracle.unpatchify: the explicit index map of einsum 'fhwpqrc->cfphqwr';
  * FastWanDiT with FAST_ATTN_IMPL="sdpa" (bf16 weights) against oracle.dit_forward
    (fp32 copy of the same weights): the whole CFG noise prediction.
The HIP ("hip") backend of the same code runs in tests/test_gpu_dit.py.
"""
import copy

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
