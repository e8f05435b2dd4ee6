"""GPU: the block and DiT forward with the HIP attention backend (FAST_ATTN_IMPL="hip")
and the fused pointwise chain (FAST_POINTWISE_IMPL="hip").

  * tiny DiT (head_dim 128, 2 layers): the CFG noise prediction against the fp32 CPU
    oracle (oracle.dit_forward), and against the reference-shaped path (torch SDPA and the
    eager pointwise ops);
  * one full-width WanAttentionBlock (dim 3072, 24 heads, ffn 14336) against the fp32 CPU
    oracle (oracle.block_forward) at a short sequence, and at the full L=7854 (config D)
    against the reference-shaped path on the GPU;
  * the fused pointwise chain against the eager one with the same attention kernels;
  * the patch-embedding GEMM against the Conv3d it replaces, and the FFN's GELU epilogue
    being the tanh form of nn.GELU(approximate="tanh");
  * masked cross-attention (per-sample text lengths) through the whole block.
Tolerances are rel-RMS: bf16 weights and activations against fp32 arithmetic.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TINY = dict(dim=256, ffn_dim=512, num_heads=2, num_layers=2, in_dim=4, out_dim=4, text_dim=64,
            freq_dim=32)


def _block_inputs(C, grid, Lc, seed):
    g = torch.Generator().manual_seed(seed)
    L = grid[0] * grid[1] * grid[2]
    x = torch.randn(2, L, C, generator=g).to(torch.bfloat16)
    e0 = (torch.randn(1, grid[0], 6, C, generator=g) * 0.1).to(torch.bfloat16)
    ctx = (torch.randn(2, Lc, C, generator=g)).to(torch.bfloat16)
    return x, e0, ctx


def test_tiny_dit_hip_vs_oracle(W):
    cfg = W.model.WanConfig(**TINY)
    m = W.model.random_model(cfg, device=DEV, std=0.05, seed=0)
    grid = (3, 4, 5)
    g = torch.Generator().manual_seed(2)
    latent = torch.randn(4, 3, 8, 10, generator=g)
    ctx_c, ctx_n = torch.randn(1, 7, 64, generator=g), torch.randn(1, 7, 64, generator=g)
    outs = {}
    for impl in ("hip", "sdpa"):
        fast = W.fast_dit.FastWanDiT(m, grid, 5.0, attn_impl=impl, cross_impl=impl,
                                     pointwise_impl="hip" if impl == "hip" else "eager")
        fast.set_context(ctx_c.to(DEV), ctx_n.to(DEV))
        outs[impl] = fast(latent.to(DEV), torch.tensor(700)).float().cpu()
    m32 = copy.deepcopy(m).float().cpu()
    m32.freqs = m.freqs
    want = ref.dit_forward(m32, latent, 700, ctx_c, ctx_n, grid, 5.0)
    e_hip, e_sdpa = ref.rel_rms(outs["hip"], want), ref.rel_rms(outs["sdpa"], want)
    print(f"tiny DiT rel_rms vs fp32 oracle: hip {e_hip:.3e}, sdpa {e_sdpa:.3e}")
    assert torch.isfinite(outs["hip"]).all()
    assert e_hip < 3e-2 and e_hip < 1.5 * e_sdpa + 5e-3


def test_denoise_never_makes_the_host_wait(W):
    """The denoising loop (DiT forwards, UniPC steps on the device, the image-latent blend)
    issues nothing that makes the host wait for the GPU: torch's sync debug mode raises on
    any such operation.  The latent is the same as with the mode off."""
    cfg = W.model.WanConfig(**TINY)
    m = W.model.random_model(cfg, device=DEV, std=0.05, seed=0)
    grid = (3, 4, 5)
    g = torch.Generator().manual_seed(3)
    latent = torch.randn(4, 3, 8, 10, generator=g).to(DEV)
    image = torch.randn(4, 1, 8, 10, generator=g).to(DEV)
    ctx_c, ctx_n = torch.randn(1, 7, 64, generator=g), torch.randn(1, 7, 64, generator=g)
    fast = W.fast_dit.FastWanDiT(m, grid, 5.0, attn_impl="hip", cross_impl="hip", pointwise_impl="hip")
    fast.set_context(ctx_c.to(DEV), ctx_n.to(DEV))
    free = W.fast_dit.denoise(fast, latent, 4, 5.0, image_latent=image)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        watched = W.fast_dit.denoise(fast, latent, 4, 5.0, image_latent=image)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert torch.isfinite(watched.float()).all()
    assert torch.equal(watched, free)


def _full_block(W, seed=0):
    cfg = W.model.WanConfig()
    m = W.model.random_model(cfg, num_layers=1, device=DEV, seed=seed)
    return m


def test_full_width_block_vs_oracle_short_sequence(W):
    """Config D block (dim 3072, ffn 14336) at L = 3*6*8 against the fp32 CPU oracle."""
    m = _full_block(W)
    blk = m.blocks[0]
    grid = (3, 6, 8)
    x, e0, ctx = _block_inputs(3072, grid, 40, 1)
    fb = W.fast_dit._FastBlock(blk, grid[0], "hip", "hip")
    cos, sin = W.rope.rope_tables(m.freqs, grid, 128, DEV)
    ck, cv = W.fast_dit._FastCrossKV(blk, "hip")(ctx.to(DEV))
    got = fb(x.to(DEV), e0.to(DEV), cos, sin, ck, cv).float().cpu()
    b32 = copy.deepcopy(blk).float().cpu()
    ck32 = ref._rms32(ref._lin32(ctx.float(), b32.cross_attn.k), b32.cross_attn.norm_k).view(2, 40, 24, 128)
    cv32 = ref._lin32(ctx.float(), b32.cross_attn.v).view(2, 40, 24, 128)
    want = ref.block_forward(b32, x.float(), e0.float(), cos.cpu(), sin.cpu(), ck32, cv32, grid[0])
    e = ref.rel_rms(got, want)
    print(f"block (L=144) rel_rms vs fp32 oracle: {e:.3e}")
    assert torch.isfinite(got).all() and e < 1e-2


@pytest.mark.parametrize("lens", [None, (77, 512)])
def test_config_d_block_hip_vs_sdpa(W, lens):
    """One WanAttentionBlock at 704x544x81 (L=7854, 21 frames) with both backends."""
    m = _full_block(W, seed=3)
    blk = m.blocks[0]
    grid = (21, 17, 22)
    x, e0, ctx = _block_inputs(3072, grid, 512, 4)
    # the block's per-frame modulation uses two timestep values: frame 0 (t=0) and the rest
    e0[:, 1:] = e0[:, 1:2]
    cos, sin = W.rope.rope_tables(m.freqs, grid, 128, DEV)
    sk = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    outs = {}
    for impl in ("hip", "sdpa"):
        fb = W.fast_dit._FastBlock(blk, grid[0], impl, impl, "hip" if impl == "hip" else "eager")
        ck, cv = W.fast_dit._FastCrossKV(blk, impl)(ctx.to(DEV))
        outs[impl] = fb(x.to(DEV), e0.to(DEV), cos, sin, ck, cv, sk).float()
    e = ref.rel_rms(outs["hip"].cpu(), outs["sdpa"].cpu())
    print(f"config D block lens={lens}: rel_rms hip vs sdpa {e:.3e}")
    assert torch.isfinite(outs["hip"]).all() and e < 1e-2


@pytest.mark.parametrize("grid", [(3, 6, 8), (21, 17, 22)])
def test_fused_pointwise_matches_eager(W, grid):
    """The same block with the four fused adaLN passes and the GELU epilogue vs the eager ops:
    the only differences are bf16 rounding (LayerNorm sum order, GELU before the rounding)."""
    m = _full_block(W, seed=5)
    blk = m.blocks[0]
    x, e0, ctx = _block_inputs(3072, grid, 512, 6)
    e0[:, 1:] = e0[:, 1:2]
    cos, sin = W.rope.rope_tables(m.freqs, grid, 128, DEV)
    ck, cv = W.fast_dit._FastCrossKV(blk, "hip")(ctx.to(DEV))
    outs = {pw: W.fast_dit._FastBlock(blk, grid[0], "hip", "hip", pw)(x.to(DEV), e0.to(DEV), cos, sin, ck, cv).float()
            for pw in ("hip", "eager")}
    e = ref.rel_rms(outs["hip"].cpu(), outs["eager"].cpu())
    print(f"grid {grid}: fused vs eager pointwise rel_rms {e:.3e}")
    assert torch.isfinite(outs["hip"]).all() and e < 5e-3


def test_patch_gemm_matches_conv3d(W):
    cfg = W.model.WanConfig(**TINY)
    m = W.model.random_model(cfg, device=DEV, std=0.05, seed=1)
    fast = W.fast_dit.FastWanDiT(m, (3, 4, 5), 5.0)
    g = torch.Generator().manual_seed(3)
    latent = torch.randn(4, 3, 8, 10, generator=g)
    got = fast.patch(latent.to(DEV)).float().cpu()
    conv = m.patch_embedding
    want = F.conv3d(latent.bfloat16().float().unsqueeze(0), conv.weight.float().cpu(), conv.bias.float().cpu(),
                    stride=conv.stride).flatten(2).transpose(1, 2)
    assert got.shape == (2, 60, cfg.dim)
    assert torch.equal(got[0], got[1])
    assert ref.rel_rms(got[:1], want) < 5e-3


def test_ffn_gelu_epilogue_is_tanh_form(W):
    """torch._addmm_activation(use_gelu=True) (the FFN-up GEMM of the fused block) applies
    the tanh-approximate GELU of nn.GELU(approximate="tanh") (wan/modules/model.py FFN).
    Checked in fp32, where tanh and erf GELU differ by far more than the GEMM's rounding."""
    xs = torch.linspace(-5, 5, 2048, device=DEV).view(2, 1024)
    eye = torch.eye(1024, device=DEV)
    y = torch._addmm_activation(torch.zeros(1024, device=DEV), xs, eye, use_gelu=True)
    d_tanh = float((y - F.gelu(xs, approximate="tanh")).abs().max())
    d_erf = float((y - F.gelu(xs)).abs().max())
    print(f"gelu epilogue: max diff vs tanh {d_tanh:.2e}, vs erf {d_erf:.2e}")
    assert d_tanh < 1e-5 < d_erf


@pytest.mark.parametrize("dim,heads,layers", [(256, 2, 3), (3072, 24, 2)])
def test_chained_block_boundaries_bit_identical(W, dim, heads, layers):
    """FastWanDiT ends each block with one fused pass that also makes the next block's norm1
    + modulation (and, after the last block, the head's): the guided prediction equals, bit
    for bit, every block's four separate stages followed by the head's own stage, with the
    HIP attention and pointwise kernels (the full-width case at a short grid)."""
    cfg = W.model.WanConfig(**dict(TINY, dim=dim, num_heads=heads, num_layers=layers,
                                   ffn_dim=4 * dim))
    m = W.model.random_model(cfg, device=DEV, std=0.05, seed=4)
    grid = (3, 4, 5)
    g = torch.Generator().manual_seed(5)
    latent = torch.randn(4, 3, 8, 10, generator=g).to(DEV)
    ctx_c, ctx_n = (torch.randn(1, 7, 64, generator=g).to(DEV) for _ in range(2))
    fast = W.fast_dit.FastWanDiT(m, grid, 5.0, attn_impl="hip", cross_impl="hip", pointwise_impl="hip")
    fast.set_context(ctx_c, ctx_n)
    t = torch.tensor(650)
    got = fast(latent, t)
    e, e0 = fast.time_rows(t)
    x = fast.patch(latent)
    for blk, (ck, cv) in zip(fast.blocks, fast.context):
        x = blk(x, e0, fast.cos, fast.sin, ck, cv, fast.seqlen_k)
    # the head's LayerNorm + modulation as its own pass of the same kernel (torch's LayerNorm
    # may order its fp32 sums differently and flip a bf16 rounding)
    rows = W.fast_dit.head_rows(m.head, e, grid[0])
    _, h = W.ops.adaln(x, None, None, grid[0], shift_idx=0, scale_idx=1, eps=m.head.norm.eps, e_mod=rows)
    want = W.fast_dit.noise_prediction(m.head, x, e, grid, m.patch_size, m.out_dim, 5.0, h=h)
    torch.cuda.synchronize()
    print(f"chained DiT dim={dim} layers={layers}: bit-identical {torch.equal(got, want)}")
    assert torch.isfinite(got.float()).all() and torch.equal(got, want)
