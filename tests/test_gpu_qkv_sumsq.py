"""GPU: the q/k/v projection GEMM with the QK-RMSNorm sums of squares in its epilogue
(wan_qkv_proj_sumsq), and the K pass that takes those sums (wan_rms_norm_qk_sumsq).

  * out = bf16(x w^T + bias) against torch's F.linear (hipBLASLt) on the same bf16 inputs,
    within one bf16 rounding (fp32 accumulation in another order may flip a rounding), and
    against a float64 product on the host; a partial last M tile, a strided output (only
    the view's elements written), the config C shape;
  * sumsq against the sums of squares of the GEMM's own bf16 output, per 64 columns;
  * inv_rms_q and the normalised, rotated k from the sums against wan_rms_norm_qk, which
    computes them from the rows (the fp32 sum order differs: equal up to rare one-ulp flips
    before the rotation, bounded against each rotated pair's norm), and against the oracle
    (oracle.inv_rms, oracle.rms, oracle.rope) on the GEMM's own q and k;
  * a whole WanAttentionBlock with FAST_QKV_IMPL "hip" against the default "hipblaslt".
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
D = 128


def _inputs(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.02).bfloat16()
    return x, w, b


def _gemm(W, x, w, b, sq, ldo=None):
    N_, lib = W._native, W._native.lib()
    M, K = x.shape
    N = w.shape[0]
    ldo = ldo or N
    big = torch.full((M, ldo), -3.0, dtype=torch.bfloat16, device=DEV)
    ss = torch.full((sq // 64 + 1, M), -1.0, dtype=torch.float32, device=DEV)
    xd, wd, bd = (t.to(DEV) for t in (x, w, b))
    with torch.cuda.device(DEV):
        N_.check("wan_qkv_proj_sumsq", lib.wan_qkv_proj_sumsq(
            xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), big.data_ptr(), ss.data_ptr(), M, N, K, K, K,
            ldo, sq, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return big, ss, (xd, wd, bd)


@pytest.mark.parametrize("M,N,K,sq,ldo", [(300, 512, 128, 192, None), (257, 768, 3072, 512, 1024),
                                          (15708, 9216, 3072, 6144, None)])
def test_gemm_matches_linear_and_sumsq(W, M, N, K, sq, ldo):
    x, w, b = _inputs(M, N, K, M + N)
    big, ss, (xd, wd, bd) = _gemm(W, x, w, b, sq, ldo)
    out = big[:, :N]
    want = F.linear(xd, wd, bd)
    d = (out.float() - want.float()).abs()
    ulp = want.float().abs().clamp_min(2 ** -100) * 2 ** -7
    frac = float((d > 0).float().mean())
    print(f"M={M} N={N} K={K}: elements differing from hipBLASLt {frac:.2e}, max {float((d / ulp).max()):.2f} ulp")
    assert bool((d <= ulp).all()) and frac < 1e-2
    if ldo is not None:
        assert bool((big[:, N:] == -3.0).all())
    # per-64-column sums of squares of the GEMM's own bf16 output; rows past sq untouched
    o = out.float()[:, :sq].reshape(M, sq // 64, 64)
    want_ss = o.pow(2).sum(-1).t()
    assert torch.allclose(ss[:sq // 64], want_ss, rtol=1e-5, atol=1e-30)
    assert bool((ss[sq // 64:] == -1.0).all())
    if M * N * K <= 1e9:
        # float64 product on the host: within bf16 rounding of the output
        exact = (x.double() @ w.double().t() + b.double())
        assert ref.rel_rms(out.cpu(), exact) < 2 ** -8


@pytest.mark.parametrize("grid", [(3, 5, 7), (21, 17, 22)])
def test_qk_prep_from_sums(W, grid):
    """The K pass from the GEMM's sums against the K pass from the rows (config C width)."""
    N_, lib = W._native, W._native.lib()
    B, H = 2, 24
    L = grid[0] * grid[1] * grid[2]
    C = H * D
    g = torch.Generator().manual_seed(9)
    h = torch.randn(B * L, C, generator=g).bfloat16()
    w = (torch.randn(3 * C, C, generator=g) * 0.02).bfloat16()
    bias = (torch.randn(3 * C, generator=g) * 0.02).bfloat16()
    big, ss, _ = _gemm(W, h, w, bias, 2 * C)
    qkv = big.view(B, L, 3 * C)
    q, k = qkv[..., :C].view(B, L, H, D), qkv[..., C:2 * C].view(B, L, H, D)
    gk = (1 + torch.rand(C, generator=g)).bfloat16().to(DEV)
    cos, sin = (t.to(DEV) for t in W.rope.rope_tables(W.rope.wan_freqs(D), grid, D))
    s = torch.cuda.current_stream().cuda_stream
    inv1, inv2 = (torch.empty(B * L, dtype=torch.float32, device=DEV) for _ in range(2))
    k1, k2 = (torch.empty(B, L, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    ssc = ss[:4 * H].contiguous()
    with torch.cuda.device(DEV):
        N_.check("sumsq", lib.wan_rms_norm_qk_sumsq(N_.tensor4(k), k1.data_ptr(), B, L, H, D, gk.data_ptr(),
                                                    1e-6, cos.data_ptr(), sin.data_ptr(), ssc.data_ptr(),
                                                    inv1.data_ptr(), s))
        N_.check("rows", lib.wan_rms_norm_qk(N_.tensor4(q), N_.tensor4(k), k2.data_ptr(), B, L, H, D,
                                             gk.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(),
                                             inv2.data_ptr(), s))
    torch.cuda.synchronize()
    assert torch.allclose(inv1, inv2, rtol=2e-6, atol=0)
    d = (k1.float() - k2.float()).abs()
    # a one-ulp flip of bf16(k * inv) becomes up to two ulps after * gamma (gamma in [1, 2)),
    # plus that product's own rounding: at most ~4 ulps of the value, measured against the
    # rotated pair's norm (the rotation preserves it; one output of a pair may have cancelled)
    pair = k2.float().view(B, L, H, D // 2, 2).pow(2).sum(-1).sqrt().repeat_interleave(2, -1).view(B, L, H, D)
    ulp = pair.clamp_min(2 ** -100) * 2 ** -7
    frac = float((d > 0).float().mean())
    print(f"grid {grid}: k-hat elements differing {frac:.2e}, max {float((d / ulp).max()):.2f} ulp of the pair norm")
    assert bool((d <= 4 * ulp).all()) and frac < 1e-2

    # ... and both against the oracle on the GEMM's own q and k: the q statistic
    # 1/sqrt(mean(q^2) + eps) (oracle.inv_rms) and k-hat = rope(rms(k) * gamma_k)
    # (oracle.rms, oracle.rope: the reference's rounding points, models/fast_dit.py:134-169)
    qh, kh = q.cpu().reshape(B, L, C), k.cpu().reshape(B, L, C)
    inv_want = ref.inv_rms(qh).reshape(-1)
    ei = float(((inv1.cpu() - inv_want).abs() / inv_want).max())
    print(f"grid {grid}: inv_rms_q from the sums vs oracle.inv_rms: max rel {ei:.2e}")
    assert ei <= 2e-6
    cos_h, sin_h = ref.rope_tables(ref.wan_freqs(D), grid, D)
    k_want = ref.rope(ref.rms(kh, gk.cpu()).view(B, L, H, D), cos_h, sin_h)
    d = (k1.cpu().float() - k_want.float()).abs()
    pair = k_want.float().view(B, L, H, D // 2, 2).pow(2).sum(-1).sqrt().repeat_interleave(2, -1).view(B, L, H, D)
    ulp = pair.clamp_min(2 ** -100) * 2 ** -7
    frac = float((d > 0).float().mean())
    print(f"grid {grid}: k-hat from the sums vs the oracle: differing {frac:.2e}, "
          f"max {float((d / ulp).max()):.2f} ulp of the pair norm")
    assert bool((d <= 4 * ulp).all()) and frac < 1e-2


def test_block_with_qkv_sumsq_matches_default(W):
    m = W.model.random_model(W.model.WanConfig(), num_layers=1, device=DEV, seed=11)
    blk = m.blocks[0]
    grid = (21, 17, 22)
    L = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, L, 3072, generator=g).bfloat16().to(DEV)
    e0 = (torch.randn(1, grid[0], 6, 3072, generator=g) * 0.1).bfloat16().to(DEV)
    ctx = torch.randn(2, 512, 3072, generator=g).bfloat16().to(DEV)
    cos, sin = W.rope.rope_tables(m.freqs, grid, 128, DEV)
    ck, cv = W.fast_dit.cross_kv(blk, ctx, "hip")
    outs = {impl: W.fast_dit._FastBlock(blk, grid[0], "hip", "hip", "hip", impl)(x, e0, cos, sin, ck, cv).float()
            for impl in ("hipblaslt", "hip")}
    e = ref.rel_rms(outs["hip"].cpu(), outs["hipblaslt"].cpu())
    print(f"block with the sums-of-squares GEMM vs hipBLASLt projection: rel_rms {e:.3e}")
    assert torch.isfinite(outs["hip"]).all() and e < 1e-3
