"""GPU parity of the HIP attention path against the CPU oracle (oracle/ref.py).

Tolerances (rel-RMS = ||y - y_ref|| / ||y_ref||, scripts/validate/attn_bench.py:114-115):
  * vs the fp32 CPU SDPA on the same prepared (bf16) q, k, v:  <= 1e-2 (the stated bar);
    measured values are ~2e-3 and the tests assert <= 5e-3 where noted;
  * vs the reference's bf16 CPU path (same rounding points):   <= 2^-7 (a couple of bf16 ulps);
  * vs the float64 golden fixtures (no intermediate rounding): <= 1e-2;
  * RoPE alone: bit-exact; RMSNorm alone: equal except where the fp32 sum order
    flips one bf16 rounding (<= 1 ulp, on < 1% of elements).
Full-size configs (L=7854) are checked on every head against the oracle and through
size-independent properties (constant V, masked keys); the long-key regime (about 12,000
keys, where the reference's NST kernel works in 8,192-key sections) on sampled heads.
"""
import math

import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu

D = 128
SCALE = D ** -0.5
DEV = torch.device("cuda:0")
TOL_FP32 = 1e-2
TOL_BF16 = 2 ** -7


def _bf(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _gammas(n, seed, peaky):
    g = torch.Generator().manual_seed(seed)
    if not peaky:
        return torch.ones(n, dtype=torch.bfloat16)
    # 1 + |N(0,1)| * s: a few channels dominate, as trained QK-norm gammas do
    return (1 + torch.randn(n, generator=g).abs() * 1.5).to(torch.bfloat16)


def _prepared(q, k, gq, gk, grid):
    """Oracle q, k after QK-RMSNorm and RoPE (bf16, the reference's rounding points)."""
    B, L, H, _ = q.shape
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    qn, kn = ref.rms_qk(q.reshape(B, L, H * D), k.reshape(B, L, H * D), gq, gk)
    return ref.rope(qn.view(B, L, H, D), cos, sin), ref.rope(kn.view(B, L, H, D), cos, sin), cos, sin


def _d(*ts):
    return [t.to(DEV) for t in ts]


# ---------------------------------------------------------------------------
# golden fixtures (float64, tests/golden/make_golden.py)
# ---------------------------------------------------------------------------

def test_golden_self_fused(W, golden):
    q, k, v = (torch.from_numpy(golden[f"self_{n}"]).bfloat16() for n in "qkv")
    gq, gk = torch.from_numpy(golden["self_gq"]).bfloat16(), torch.from_numpy(golden["self_gk"]).bfloat16()
    grid = tuple(int(x) for x in golden["self_grid"])
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    out = W.ops.self_attn_fused(*_d(q, k, v, gq, gk), 1e-6, *_d(cos, sin), SCALE).cpu()
    assert ref.rel_rms(out, torch.from_numpy(golden["self_out"])) <= TOL_FP32
    assert ref.rel_rms(out, ref.self_attn_path(q, k, v, gq, gk, cos, sin)) <= TOL_BF16


def test_golden_cross_fused(W, golden):
    q, ck, cv = (torch.from_numpy(golden[f"cross_{n}"]).bfloat16() for n in "qkv")
    gq = torch.from_numpy(golden["cross_gq"]).bfloat16()
    lens = torch.from_numpy(golden["cross_lens"]).int()
    out = W.ops.cross_attn_fused(*_d(q, ck, cv, gq), 1e-6, lens.to(DEV), SCALE).cpu()
    assert ref.rel_rms(out, torch.from_numpy(golden["cross_out"])) <= TOL_FP32


def test_golden_plain_masked(W, golden):
    q, k, v = (torch.from_numpy(golden[f"plain_{n}"]).bfloat16() for n in "qkv")
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, int(golden["plain_len"])).cpu()
    assert ref.rel_rms(out, torch.from_numpy(golden["plain_out"])) <= TOL_FP32


# ---------------------------------------------------------------------------
# plain attention at ragged sizes (tails of the 64-key tile and 128-row block)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,Lq,Lk,H,actual", [
    (1, 1, 1, 1, 0),
    (1, 5, 3, 2, 0),
    (1, 64, 64, 1, 0),
    (2, 63, 65, 3, 0),
    (1, 129, 200, 2, 129),
    (2, 257, 77, 2, 0),
    (1, 300, 300, 2, 1),
    (1, 1000, 1000, 1, 999),
])
def test_plain_self_ragged(W, B, Lq, Lk, H, actual):
    seed = B * 1000 + Lq + 7 * Lk + H
    q, k, v = _bf((B, Lq, H, D), seed), _bf((B, Lk, H, D), seed + 1), _bf((B, Lk, H, D), seed + 2)
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, actual).cpu()
    n = actual if actual > 0 else Lk
    want32 = ref.sdpa(q.float(), k.float(), v.float(), seqlen_k=n)
    want16 = ref.sdpa(q, k, v, seqlen_k=n)
    assert torch.isfinite(out.float()).all()
    assert ref.rel_rms(out, want32) <= 5e-3
    assert ref.rel_rms(out, want16) <= TOL_BF16


@pytest.mark.parametrize("pattern,actual,Lk", [
    ("rising", 0, 1000), ("falling", 0, 1000), ("jumps", 0, 1000), ("jumps", 937, 1000),
    # more than 1024 keys: the 8-wave kernel with its ring of four K/V tiles; 20 tiles leave
    # the three-step remainder after the ring's groups of four, 2000 keys a partial last tile
    ("rising", 0, 1280), ("falling", 0, 1280), ("jumps", 0, 1280), ("jumps", 0, 2000),
    ("rising", 1990, 2000), ("jumps", 1217, 2000)])
def test_large_logit_swings(W, pattern, actual, Lk):
    """Logits whose level moves by ~10-60 natural units between 64-key tiles (up to ~200:
    exp overflows without a reference max).  Exercises the exact-max rescale of O and l,
    which runs only when a tile's sum of p exceeds its bound."""
    B, Lq, H = 1, 96, 2
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, Lq, H, D, generator=g) * 0.3
    q[..., 0] = 1.0 + 0.1 * torch.randn(B, Lq, H, generator=g)
    k = torch.randn(B, Lk, H, D, generator=g) * 0.3
    j = torch.arange(Lk, dtype=torch.float32)
    if pattern == "rising":
        level = 0.2 * j
    elif pattern == "falling":
        level = -0.2 * j
    else:
        level = (torch.rand(Lk // 64 + 1, generator=g) * 120 - 60).repeat_interleave(64)[:Lk]
    k[..., 0] = (level / SCALE).view(1, Lk, 1)
    v = torch.randn(B, Lk, H, D, generator=g)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, actual).cpu()
    n = actual if actual > 0 else Lk
    want = torch.from_numpy(ref.brute_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                                SCALE, n)).float()
    e = ref.rel_rms(out, want)
    print(f"{pattern} actual={actual}: rel_rms vs float64 {e:.3e}")
    assert torch.isfinite(out.float()).all() and e <= 5e-3


@pytest.mark.parametrize("Lq,Lk,actual", [
    (300, 1280, 0),      # 20 full tiles: ring groups of four plus the three-step remainder
    (300, 1344, 0),      # 21 tiles: no remainder step before the last tile
    (300, 1281, 0),      # 21 tiles, the last holds one key
    (257, 2048, 0),      # 32 full tiles
    (257, 2048, 1),      # one key
    (257, 2048, 50),     # one partial tile
    (257, 2048, 64),     # one full tile
    (257, 2048, 128),    # two tiles
    (257, 2048, 192),    # three tiles
    (257, 2048, 250),    # four tiles, the last partial
    (513, 1025, 1025),   # the smallest key count of the 8-wave kernel
])
def test_eight_wave_kernel_tile_counts(W, Lq, Lk, actual):
    """Key counts above 1024 select the 8-wave kernel (256 query rows per workgroup, a ring
    of four K and four V tiles, a barrier every second tile).  Every remainder of the ring
    (tile counts 1-4 and 20, 21 = 0 and 1 mod 4, with 22/23 covered by L=1080 and 7854),
    full and partial last tiles, against the fp32 and bf16 oracle."""
    B, H = 2, 2
    seed = 5000 + Lq + Lk + actual
    q, k, v = _bf((B, Lq, H, D), seed), _bf((B, Lk, H, D), seed + 1), _bf((B, Lk, H, D), seed + 2)
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, actual).cpu()
    n = actual if actual > 0 else Lk
    assert torch.isfinite(out.float()).all()
    assert ref.rel_rms(out, ref.sdpa(q.float(), k.float(), v.float(), seqlen_k=n)) <= 5e-3
    assert ref.rel_rms(out, ref.sdpa(q, k, v, seqlen_k=n)) <= TOL_BF16


@pytest.mark.parametrize("fused", [False, True])
def test_eight_wave_per_sample_lengths(W, fused):
    """Per-sample key lengths and the in-kernel Q RMSNorm with more than 1024 keys (the
    8-wave kernel): lengths 1, 130, 2000 and 0 in one batch, NaN in V and huge K past each
    length, against the oracle; the length-0 sample is all zeros."""
    B, H, Lq, Lk = 4, 3, 300, 2048
    lens = [1, 130, 2000, 0]
    q, ck, cv = _bf((B, Lq, H, D), 301), _bf((B, Lk, H, D), 302), _bf((B, Lk, H, D), 303)
    gq = _gammas(H * D, 304, True)
    ck2, cv2 = ck.clone(), cv.clone()
    for b, n in enumerate(lens):
        ck2[b, n:] = _bf((Lk - n, H, D), 310 + b, std=50.0)
        cv2[b, n:] = float("nan")
    sk = torch.tensor(lens, dtype=torch.int32).to(DEV)
    if fused:
        out = W.ops.cross_attn_fused(*_d(q, ck2, cv2, gq), 1e-6, sk, SCALE).cpu()
        qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    else:
        out = W.ops.cross_attn(*_d(q, ck2, cv2), sk, SCALE).cpu()
        qn = q
    assert torch.isfinite(out.float()).all()
    assert torch.count_nonzero(out[3]) == 0
    want = ref.sdpa(qn.float(), ck.float(), cv.float(), seqlen_k=lens)
    for b in range(3):
        e = ref.rel_rms(out[b], want[b])
        print(f"fused={fused} len={lens[b]}: rel_rms vs fp32 {e:.3e}")
        assert e <= 5e-3


def test_single_key_returns_its_value(W):
    q, k, v = _bf((2, 77, 3, D), 1), _bf((2, 9, 3, D), 2), _bf((2, 9, 3, D), 3)
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, 1).cpu()
    assert torch.equal(out, v[:, :1].expand(-1, 77, -1, -1))


def test_strided_views(W):
    """Projections are [B, L, 3072] tensors viewed as [B, L, 24, 128]; also a batch-inner layout."""
    B, L, H = 2, 150, 24
    x = _bf((B, L, 3 * H * D), 5)
    q, k, v = x[..., :H * D].view(B, L, H, D), x[..., H * D:2 * H * D].view(B, L, H, D), x[..., 2 * H * D:].view(B, L, H, D)
    out = W.ops.flash_self_attn(*_d(q, k, v), SCALE, 0).cpu()
    assert ref.rel_rms(out, ref.sdpa(q.float(), k.float(), v.float())) <= 5e-3
    kb = _bf((L, B, H, D), 6).to(DEV).transpose(0, 1)  # batch stride H*D, token stride B*H*D
    qd, vd = q.contiguous().to(DEV), v.contiguous().to(DEV)
    out2 = W.ops.flash_self_attn(qd, kb, vd, SCALE, 0).cpu()
    assert ref.rel_rms(out2, ref.sdpa(q.float(), kb.cpu().float(), v.float())) <= 5e-3


# ---------------------------------------------------------------------------
# fused QK-RMSNorm + RoPE self-attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("peaky", [False, True])
def test_config_a_fused(W, peaky):
    """B=2, L=1080 (grid 6x12x15), 24 heads: the whole output against the oracle."""
    B, H, grid = 2, 24, (6, 12, 15)
    L = grid[0] * grid[1] * grid[2]
    q, k, v = _bf((B, L, H, D), 11), _bf((B, L, H, D), 12), _bf((B, L, H, D), 13)
    gq, gk = _gammas(H * D, 14, peaky), _gammas(H * D, 15, peaky)
    qr, kr, cos, sin = _prepared(q, k, gq, gk, grid)
    out = W.ops.self_attn_fused(*_d(q, k, v, gq, gk), 1e-6, *_d(cos, sin), SCALE).cpu()
    assert torch.isfinite(out.float()).all()
    want32 = ref.sdpa(qr.float(), kr.float(), v.float())
    e32 = ref.rel_rms(out, want32)
    e16 = ref.rel_rms(out, ref.sdpa(qr, kr, v))
    print(f"config A peaky={peaky}: rel_rms vs fp32 {e32:.3e}, vs bf16 path {e16:.3e}")
    assert e32 <= 5e-3 and e16 <= TOL_BF16
    # Against the fully fp32 path (norm and rope without bf16 rounding) the kernel is within
    # the stated bar, or, where the reference's own bf16 rounding of q and k already costs
    # more than that (peaky gammas: large logits), no further from it than the reference is.
    full32 = ref.self_attn_path(q.float(), k.float(), v.float(), gq.float(), gk.float(), cos, sin)
    e_ref = ref.rel_rms(ref.sdpa(qr, kr, v), full32)
    e_out = ref.rel_rms(out, full32)
    print(f"config A peaky={peaky}: vs exact fp32 math: kernel {e_out:.3e}, reference bf16 path {e_ref:.3e}")
    assert e_out <= max(TOL_FP32, 1.1 * e_ref)


def test_fused_equals_standalone_ops(W):
    """fused(q, k, v) == attention(rope(rms(q)), rope(rms(k)), v) from the standalone kernels."""
    B, H, grid = 2, 6, (3, 5, 7)
    L = grid[0] * grid[1] * grid[2]
    q, k, v = _bf((B, L, H, D), 21), _bf((B, L, H, D), 22), _bf((B, L, H, D), 23)
    gq, gk = _gammas(H * D, 24, True), _gammas(H * D, 25, True)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    qd, kd, vd, gqd, gkd, cd, sd = _d(q, k, v, gq, gk, cos, sin)
    fused = W.ops.self_attn_fused(qd, kd, vd, gqd, gkd, 1e-6, cd, sd, SCALE)
    qh = W.ops.rope(W.ops.rms_norm(qd, gqd, 1e-6), cd, sd)
    kh = W.ops.rope(W.ops.rms_norm(kd, gkd, 1e-6), cd, sd)
    plain = W.ops.flash_self_attn(qh, kh, vd, SCALE, 0)
    assert torch.equal(fused, plain)


def test_rms_norm_qk_equals_two_passes(W):
    """wan_rms_norm_qk (one launch) == wan_rms_norm(q: statistics) + wan_rms_norm(k: norm+rope),
    bit for bit, on strided [B, L, 3072] views at the config C width."""
    N = W._native
    lib = N.lib()
    B, H, grid = 2, 24, (3, 7, 9)
    L = grid[0] * grid[1] * grid[2]
    x = _bf((B, L, 3 * H * D), 31).to(DEV)
    q, k = x[..., :H * D].view(B, L, H, D), x[..., H * D:2 * H * D].view(B, L, H, D)
    gk = _gammas(H * D, 32, True).to(DEV)
    cos, sin = (t.to(DEV) for t in ref.rope_tables(ref.wan_freqs(D), grid, D))
    s = torch.cuda.current_stream().cuda_stream
    inv1, inv2 = (torch.empty(B * L, dtype=torch.float32, device=DEV) for _ in range(2))
    k1, k2 = (torch.empty(B, L, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    N.check("qk", lib.wan_rms_norm_qk(N.tensor4(q), N.tensor4(k), k1.data_ptr(), B, L, H, D,
                                      gk.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(),
                                      inv1.data_ptr(), s))
    N.check("q", lib.wan_rms_norm(N.tensor4(q), None, B, L, H, D, None, 1e-6, None, None,
                                  inv2.data_ptr(), s))
    N.check("k", lib.wan_rms_norm(N.tensor4(k), k2.data_ptr(), B, L, H, D, gk.data_ptr(), 1e-6,
                                  cos.data_ptr(), sin.data_ptr(), None, s))
    torch.cuda.synchronize()
    assert torch.equal(inv1, inv2) and torch.equal(k1, k2)
    want = ref.inv_rms(q.cpu().reshape(B, L, H * D).float())
    assert torch.allclose(inv1.cpu().view(B, L), want.view(B, L), rtol=1e-5)


def test_rope_bit_exact(W):
    B, H, grid = 2, 24, (4, 6, 8)
    L = grid[0] * grid[1] * grid[2]
    x = _bf((B, L, H, D), 31, std=3.0)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    out = W.ops.rope(*_d(x, cos, sin)).cpu()
    assert torch.equal(out, ref.rope(x, cos, sin))


def test_rms_norm_matches_reference_rounding(W):
    B, L, H = 2, 333, 24
    x = _bf((B, L, H, D), 41, std=2.0)
    g = _gammas(H * D, 42, True)
    out = W.ops.rms_norm(*_d(x, g), 1e-6).cpu()
    want = ref.rms(x.reshape(B, L, H * D), g).view(B, L, H, D)
    diff = (out.float() - want.float()).abs()
    ulp = want.float().abs().clamp_min(1e-30) * 2 ** -7
    assert bool((diff <= ulp).all())
    assert float((diff > 0).float().mean()) < 1e-2
    inv = W.ops.rms_inv(x.to(DEV), 1e-6).cpu()
    assert torch.allclose(inv, ref.inv_rms(x.reshape(B, L, H * D)), rtol=1e-6)


# ---------------------------------------------------------------------------
# cross-attention with per-sample key lengths (config B)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("lens", [None, (16, 512), (137, 289), (1, 64), (0, 511)])
def test_cross_config_b(W, lens):
    B, H, Lq, Lk = 2, 24, 7854, 512
    q, ck, cv = _bf((B, Lq, H, D), 51), _bf((B, Lk, H, D), 52), _bf((B, Lk, H, D), 53)
    gq = _gammas(H * D, 54, True)
    sk = None if lens is None else torch.tensor(lens, dtype=torch.int32)
    out = W.ops.cross_attn_fused(*_d(q, ck, cv, gq), 1e-6, None if sk is None else sk.to(DEV), SCALE).cpu()
    qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    want = ref.sdpa(qn.float(), ck.float(), cv.float(), seqlen_k=None if lens is None else list(lens))
    assert torch.isfinite(out.float()).all()
    if lens is not None and 0 in lens:
        b0 = lens.index(0)
        assert torch.count_nonzero(out[b0]) == 0
        keep = [b for b in range(B) if b != b0]
        out, want = out[keep], want[keep]
    assert ref.rel_rms(out, want) <= 5e-3


@pytest.mark.parametrize("lens", ["drawn", (512, 512)])
def test_cross_config_b_text_recipe(W, lens):
    """Config B with its K/V built as the pipeline builds them: a [2, 512, 4096] N(0,1) text
    context through the DiT's text embedding (Linear, tanh-GELU, Linear; std-0.02 weights),
    then one block's lin_k + RMSNorm and lin_v (models/fast_dit.py:464-477), on the device in
    bf16 by the product; seqlen_k drawn from U{16..512} (and both 512, the reference
    pipeline's unmasked case).  K/V against the fp32 chain on the host, then the attention
    against the fp32 SDPA on the product's own K/V."""
    import copy
    B, H, Lq, Lc = 2, 24, 7854, 512
    m = W.model.random_model(W.model.WanConfig(), num_layers=1, device=DEV, seed=61)
    blk = m.blocks[0]
    g = torch.Generator().manual_seed(62)
    ctx = torch.randn(B, Lc, 4096, generator=g).bfloat16()
    ck, cv = W.fast_dit.cross_kv(blk, m.text_embedding(ctx.to(DEV)), "hip")
    host_te = copy.deepcopy(m.text_embedding).float().cpu()
    host_blk = copy.deepcopy(blk).float().cpu()
    ck32, cv32 = ref.cross_kv(host_blk, ref.text_context(host_te, ctx), H, D)
    e_k, e_v = ref.rel_rms(ck.cpu(), ck32), ref.rel_rms(cv.cpu(), cv32)
    print(f"text recipe: ck {e_k:.2e}, cv {e_v:.2e} from the fp32 chain")
    assert e_k < 1e-2 and e_v < 1e-2
    sk = torch.randint(16, Lc + 1, (B,), generator=g, dtype=torch.int32) if lens == "drawn" \
        else torch.tensor(lens, dtype=torch.int32)
    q = _bf((B, Lq, H, D), 63)
    gq = _gammas(H * D, 64, True)
    out = W.ops.cross_attn_fused(*_d(q), ck, cv, gq.to(DEV), 1e-6, sk.to(DEV), SCALE).cpu()
    qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    want = ref.sdpa(qn.float(), ck.cpu().float(), cv.cpu().float(), seqlen_k=sk.tolist())
    e = ref.rel_rms(out, want)
    print(f"seqlen_k {sk.tolist()}: attention rel_rms {e:.2e} vs the fp32 SDPA")
    assert torch.isfinite(out.float()).all() and e <= 5e-3


@pytest.mark.parametrize("fused,B,H", [(True, 3, 64), (False, 3, 64), (True, 9, 8), (False, 9, 8)])
def test_cross_lengths_table_limits(W, fused, B, H):
    """The persistent short-key kernel keeps the query gammas (H x 128) and the key lengths
    (B) in a 16 KB LDS table: at 64 heads with the fused Q norm they do not fit and the
    plain kernel runs instead; without the norm (no gammas) or at 8 heads they fit.  Both
    against the oracle, with lengths 0, 1, a partial tile and the full 512."""
    Lq, Lk = 300, 512
    lens = ([0, 1, 512, 130, 64, 511, 2, 200, 17] * 2)[:B]
    q, ck, cv = _bf((B, Lq, H, D), 501 + H), _bf((B, Lk, H, D), 502 + H), _bf((B, Lk, H, D), 503 + H)
    gq = _gammas(H * D, 504, True)
    sk = torch.tensor(lens, dtype=torch.int32).to(DEV)
    if fused:
        out = W.ops.cross_attn_fused(*_d(q, ck, cv, gq), 1e-6, sk, SCALE).cpu()
        qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    else:
        out = W.ops.cross_attn(*_d(q, ck, cv), sk, SCALE).cpu()
        qn = q
    want = ref.sdpa(qn.float(), ck.float(), cv.float(), seqlen_k=lens)
    keep = [b for b in range(B) if lens[b] > 0]
    for b in range(B):
        if lens[b] == 0:
            assert torch.count_nonzero(out[b]) == 0
    assert torch.isfinite(out.float()).all()
    assert ref.rel_rms(out[keep], want[keep]) <= 5e-3


@pytest.mark.parametrize("fused", [False, True])
def test_persistent_cross_mixed_lengths(W, fused):
    """Per-sample key lengths select the persistent short-key kernel: each workgroup walks
    several (batch, head, 128-row block) items, fetching the next item's tiles and query
    rows while it finishes the current one.  Five samples with lengths 512, 0, 1, 130 and
    64 (full, empty, a single key, partial and exactly one tile), NaN and huge K past each
    length, 24 heads: many items per workgroup, in every order of long and short."""
    B, H, Lq, Lk = 5, 24, 1000, 512
    lens = [512, 0, 1, 130, 64]
    q, ck, cv = _bf((B, Lq, H, D), 401), _bf((B, Lk, H, D), 402), _bf((B, Lk, H, D), 403)
    gq = _gammas(H * D, 404, True)
    ck2, cv2 = ck.clone(), cv.clone()
    for b, n in enumerate(lens):
        ck2[b, n:] = _bf((Lk - n, H, D), 410 + b, std=50.0)
        cv2[b, n:] = float("nan")
    sk = torch.tensor(lens, dtype=torch.int32).to(DEV)
    if fused:
        out = W.ops.cross_attn_fused(*_d(q, ck2, cv2, gq), 1e-6, sk, SCALE).cpu()
        qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    else:
        out = W.ops.cross_attn(*_d(q, ck2, cv2), sk, SCALE).cpu()
        qn = q
    assert torch.isfinite(out.float()).all()
    assert torch.count_nonzero(out[1]) == 0
    want = ref.sdpa(qn.float(), ck.float(), cv.float(), seqlen_k=lens)
    for b in (0, 2, 3, 4):
        e = ref.rel_rms(out[b], want[b])
        print(f"fused={fused} len={lens[b]}: rel_rms vs fp32 {e:.3e}")
        assert e <= 5e-3


@pytest.mark.parametrize("B,Lq,Lk", [(2, 7854, 512), (3, 130, 77), (1, 5, 64)])
def test_persistent_equals_plain_kernel(W, B, Lq, Lk):
    """Lengths all equal to Lk (the persistent kernel) against no lengths (the plain
    short-key kernel): the same arithmetic in the same order, so the same bits; the
    small shapes have fewer items than workgroups."""
    H = 24 if Lq > 1000 else 3
    q, ck, cv = _bf((B, Lq, H, D), 501), _bf((B, Lk, H, D), 502), _bf((B, Lk, H, D), 503)
    gq = _gammas(H * D, 504, True)
    sk = torch.full((B,), Lk, dtype=torch.int32).to(DEV)
    qd, kd, vd, gd = _d(q, ck, cv, gq)
    assert torch.equal(W.ops.cross_attn_fused(qd, kd, vd, gd, 1e-6, sk, SCALE),
                       W.ops.cross_attn_fused(qd, kd, vd, gd, 1e-6, None, SCALE))
    assert torch.equal(W.ops.cross_attn(qd, kd, vd, sk, SCALE), W.ops.cross_attn(qd, kd, vd, None, SCALE))


def test_cross_masked_keys_do_not_matter(W):
    B, H, Lq, Lk = 2, 24, 1000, 512
    q, ck, cv = _bf((B, Lq, H, D), 61), _bf((B, Lk, H, D), 62), _bf((B, Lk, H, D), 63)
    lens = torch.tensor([100, 333], dtype=torch.int32)
    ck2, cv2 = ck.clone(), cv.clone()
    for b, n in enumerate(lens.tolist()):
        ck2[b, n:] = _bf((Lk - n, H, D), 64 + b, std=50.0)
        cv2[b, n:] = float("nan")
    a = W.ops.cross_attn(*_d(q, ck, cv), lens.to(DEV), SCALE)
    b = W.ops.cross_attn(*_d(q, ck2, cv2), lens.to(DEV), SCALE)
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# full size self-attention (config C, L=7854 = grid 21x17x22)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("grid", [(21, 17, 22), (21, 22, 17)])
def test_config_c_fused_all_heads(W, grid):
    """L=7854 at the pipeline's latent grid (21, 17, 22) and at the reference block bench's
    (21, 22, 17) (scripts/validate/block_bench.py:34): the same token count, other tables.
    Every one of the 24 heads of both samples against the fp32 oracle (the whole output, and
    each (batch, head) on its own so that one bad head cannot hide in the average)."""
    B, H = 2, 24
    L = grid[0] * grid[1] * grid[2]
    q, k, v = _bf((B, L, H, D), 71), _bf((B, L, H, D), 72), _bf((B, L, H, D), 73)
    gq, gk = _gammas(H * D, 74, True), _gammas(H * D, 75, True)
    qr, kr, cos, sin = _prepared(q, k, gq, gk, grid)
    out = W.ops.self_attn_fused(*_d(q, k, v, gq, gk), 1e-6, *_d(cos, sin), SCALE).cpu()
    assert torch.isfinite(out.float()).all()
    want = ref.sdpa(qr.float(), kr.float(), v.float())
    e = ref.rel_rms(out, want)
    per = torch.tensor([[ref.rel_rms(out[b, :, h], want[b, :, h]) for h in range(H)] for b in range(B)])
    print(f"config C grid {grid} all {B}x{H} heads: rel_rms vs fp32 {e:.3e}, worst head {float(per.max()):.3e}")
    assert e <= 5e-3 and float(per.max()) <= 5e-3


# ---------------------------------------------------------------------------
# long keys: past the 10,240 keys where the reference's NST kernel switches to 8,192-key
# sections with an fp32 partial output in HBM (kernels/self_attention_nst.py:45-46,96-103).
# These kernels stream any number of keys in one pass; the result must still be SDPA.
# ---------------------------------------------------------------------------

def test_long_keys_fused_self_attention(W):
    """12,000 tokens (grid 25 x 20 x 24: a partial last key tile and query block), Q/K norm
    and RoPE fused, 4 heads of both samples against the fp32 oracle."""
    B, H, grid = 2, 4, (25, 20, 24)
    L = grid[0] * grid[1] * grid[2]
    q, k, v = _bf((B, L, H, D), 171), _bf((B, L, H, D), 172), _bf((B, L, H, D), 173)
    gq, gk = _gammas(H * D, 174, True), _gammas(H * D, 175, True)
    qr, kr, cos, sin = _prepared(q, k, gq, gk, grid)
    out = W.ops.self_attn_fused(*_d(q, k, v, gq, gk), 1e-6, *_d(cos, sin), SCALE).cpu()
    assert torch.isfinite(out.float()).all()
    want = ref.sdpa(qr.float(), kr.float(), v.float())
    e = ref.rel_rms(out, want)
    e16 = ref.rel_rms(out, ref.sdpa(qr, kr, v))
    print(f"L={L} fused: rel_rms vs fp32 {e:.3e}, vs the bf16 path {e16:.3e}")
    assert e <= 5e-3 and e16 <= TOL_BF16


@pytest.mark.parametrize("Lk,actual", [(12288, 11000), (16000, 0)])
def test_long_keys_actual_seqlen(W, Lk, actual):
    """wan_flash_self_attn over 12,288 keys with actual_seqlen_k 11,000 (the NST kernel's
    padded-key semantics, kernels/self_attention_nst.py:73-78) and over 16,000 keys."""
    B, H, Lq = 1, 3, 700
    q, k, v = _bf((B, Lq, H, D), 181), _bf((B, Lk, H, D), 182), _bf((B, Lk, H, D), 183)
    n = actual or Lk
    k2, v2 = k.clone(), v.clone()
    k2[:, n:] = 1e4
    v2[:, n:] = float("nan")
    out = W.ops.flash_self_attn(*_d(q, k2, v2), SCALE, actual).cpu()
    want = ref.sdpa(q.float(), k.float(), v.float(), seqlen_k=[n] * B)
    e = ref.rel_rms(out, want)
    print(f"Lk={Lk} actual={n}: rel_rms vs fp32 {e:.3e}")
    assert torch.isfinite(out.float()).all() and e <= 5e-3


def test_config_c_constant_v(W):
    """softmax rows sum to one: a per-head constant V comes back unchanged, for every query."""
    B, H, grid = 2, 24, (21, 17, 22)
    L = grid[0] * grid[1] * grid[2]
    q, k = _bf((B, L, H, D), 81), _bf((B, L, H, D), 82)
    c = _bf((B, 1, H, D), 83)
    v = c.expand(B, L, H, D).contiguous()
    gq, gk = _gammas(H * D, 84, True), _gammas(H * D, 85, True)
    cos, sin = ref.rope_tables(ref.wan_freqs(D), grid, D)
    out = W.ops.self_attn_fused(*_d(q, k, v, gq, gk), 1e-6, *_d(cos, sin), SCALE).cpu().float()
    want = c.float().expand(B, L, H, D)
    rel = ((out - want).abs() / want.abs().clamp_min(1e-3)).max()
    assert float(rel) <= 2 ** -7


# ---------------------------------------------------------------------------
# output placement and repeatability
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,Lq,Lk,H,lens", [(2, 300, 300, 3, None), (2, 1100, 1100, 2, None),
                                            (2, 333, 77, 2, (77, 5))])
def test_output_stays_inside_its_view(W, B, Lq, Lk, H, lens):
    """The output tile is staged through LDS and written as whole row segments: into an
    output that is a strided view of a larger buffer (32 rows before and after, one head
    on either side), exactly the view's elements change.  Covers the 8-wave (1100 keys)
    and 4-wave (300, 77 keys) kernels and a partial last query block."""
    N, lib = W._native, W._native.lib()
    q, k, v = _bf((B, Lq, H, D), 91), _bf((B, Lk, H, D), 92), _bf((B, Lk, H, D), 93)
    big = torch.full((B, Lq + 64, H + 2, D), -7.0, dtype=torch.bfloat16, device=DEV)
    view = big[:, 32:32 + Lq, 1:1 + H, :]
    qd, kd, vd = _d(q, k, v)
    s = torch.cuda.current_stream().cuda_stream
    if lens is None:
        N.check("wan_flash_self_attn", lib.wan_flash_self_attn(
            N.tensor4(qd), N.tensor4(kd), N.tensor4(vd), N.tensor4(view), B, H, Lq, Lk, D, SCALE, 0, s))
    else:
        sk = torch.tensor(lens, dtype=torch.int32, device=DEV)
        N.check("wan_cross_attn", lib.wan_cross_attn(
            N.tensor4(qd), N.tensor4(kd), N.tensor4(vd), N.tensor4(view), B, H, Lq, Lk, D, SCALE,
            sk.data_ptr(), s))
    torch.cuda.synchronize()
    host = big.cpu()
    inside = torch.zeros(host.shape, dtype=torch.bool)
    inside[:, 32:32 + Lq, 1:1 + H, :] = True
    assert bool((host[~inside] == -7.0).all())
    want = ref.sdpa(q.float(), k.float(), v.float(), seqlen_k=None if lens is None else list(lens))
    assert ref.rel_rms(host[:, 32:32 + Lq, 1:1 + H, :], want) <= 5e-3


def test_repeat_calls_bit_identical(W):
    """No atomics and a fixed reduction order: repeated launches at full size return the
    same bits (a missing wait or barrier between the tile copies and their readers would
    show up here as run-to-run differences)."""
    B, H, grid = 2, 24, (21, 17, 22)
    L = grid[0] * grid[1] * grid[2]
    g = torch.Generator(device=DEV).manual_seed(95)
    q, k, v = (torch.randn(B, L, H, D, device=DEV, generator=g).to(torch.bfloat16) for _ in range(3))
    gq, gk = _d(_gammas(H * D, 96, True), _gammas(H * D, 97, True))
    cos, sin = _d(*ref.rope_tables(ref.wan_freqs(D), grid, D))
    outs = [W.ops.self_attn_fused(q, k, v, gq, gk, 1e-6, cos, sin, SCALE) for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ck, cv = k[:, :512].contiguous(), v[:, :512].contiguous()
    lens = torch.tensor([470, 123], dtype=torch.int32, device=DEV)
    outs = [W.ops.cross_attn_fused(q, ck, cv, gq, 1e-6, lens, SCALE) for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
