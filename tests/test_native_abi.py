"""The C ABI library on the CPU: it loads, exports every function include/wan_attn.h
declares, and rejects bad arguments before any device work.  No kernel is launched.
"""
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wan_attn.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wan_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = header_functions()
    for n in ("wan_flash_self_attn", "wan_cross_attn", "wan_self_attn_fused", "wan_cross_attn_fused",
              "wan_rope", "wan_rms_norm", "wan_attn_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol(W):
    lib = W._native.lib()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(W._native.SIGNATURES) == set(header_functions())


def test_abi_version(W):
    assert W._native.lib().wan_attn_abi_version() == W._native.ABI_VERSION


def test_validation_rejects_bad_arguments_without_launching(W):
    N = W._native
    lib = N.lib()
    ok = N.WanTensor(64, 24 * 128 * 16, 24 * 128, 128)
    # head_dim other than 128 is unsupported
    rc = lib.wan_flash_self_attn(ok, ok, ok, ok, 1, 24, 16, 16, 64, 0.1, 0, None)
    assert rc == 2 and "head_dim" in N.last_error()
    # misaligned pointer
    bad = N.WanTensor(66, 24 * 128 * 16, 24 * 128, 128)
    rc = lib.wan_flash_self_attn(bad, ok, ok, ok, 1, 24, 16, 16, 128, 0.1, 0, None)
    assert rc == 1 and "aligned" in N.last_error()
    # stride not a multiple of 8
    bad = N.WanTensor(64, 24 * 128 * 16, 24 * 128 + 4, 128)
    rc = lib.wan_flash_self_attn(ok, bad, ok, ok, 1, 24, 16, 16, 128, 0.1, 0, None)
    assert rc == 1 and "stride" in N.last_error()
    # token stride too large for the tile loader's 32-bit offsets
    bad = N.WanTensor(64, 24 * 128 * 16, 1 << 24, 128)
    rc = lib.wan_flash_self_attn(ok, bad, ok, ok, 1, 24, 16, 16, 128, 0.1, 0, None)
    assert rc == 2 and "token stride" in N.last_error()
    # actual_seqlen_k beyond the keys
    rc = lib.wan_flash_self_attn(ok, ok, ok, ok, 1, 24, 16, 16, 128, 0.1, 17, None)
    assert rc == 1 and "actual_seqlen_k" in N.last_error()
    # NULL operand
    rc = lib.wan_cross_attn(ok, N.WanTensor(0, 0, 0, 0), ok, ok, 1, 24, 16, 16, 128, 0.1, None, None)
    assert rc == 1 and "NULL" in N.last_error()
    # fused: workspace too small / missing tables
    rc = lib.wan_self_attn_fused(ok, ok, ok, ok, 1, 24, 16, 128, 256, 256, 1e-6, 256, 256, 0.1,
                                 256, 10, None)
    assert rc == 3 and "workspace" in N.last_error()
    rc = lib.wan_self_attn_fused(ok, ok, ok, ok, 1, 24, 16, 128, None, 256, 1e-6, 256, 256, 0.1,
                                 256, 1 << 30, None)
    assert rc == 1
    rc = lib.wan_cross_attn_fused(ok, ok, ok, ok, 1, 24, 16, 8, 128, 256, -1.0, 0.1, None, 256,
                                  1 << 30, None)
    assert rc == 1 and "eps" in N.last_error()
    # rms_norm: rotation without an output, one table missing
    rc = lib.wan_rms_norm(ok, None, 1, 16, 24, 128, 256, 1e-6, 256, 256, None, None)
    assert rc == 1 and "out" in N.last_error()
    rc = lib.wan_rms_norm(ok, 256, 1, 16, 24, 128, 256, 1e-6, 256, None, None, None)
    assert rc == 1 and "both" in N.last_error()
    rc = lib.wan_flash_attn_qnorm(ok, ok, ok, ok, 1, 24, 16, 16, 128, None, 256, None, None, 0.1,
                                  None, None)
    assert rc == 1 and "inv_rms_q" in N.last_error()
    # rms_norm_qk: both outputs are required; k's gamma is required with an output
    rc = lib.wan_rms_norm_qk(ok, ok, None, 1, 16, 24, 128, 256, 1e-6, 256, 256, 256, None)
    assert rc == 1 and "required" in N.last_error()
    rc = lib.wan_rms_norm_qk(ok, ok, 256, 1, 16, 24, 128, None, 1e-6, 256, 256, 256, None)
    assert rc == 1 and "gamma" in N.last_error()
    rc = lib.wan_rms_norm_qk(ok, ok, 256, 1, 16, 24, 64, 256, 1e-6, 256, 256, 256, None)
    assert rc == 2 and "head_dim" in N.last_error()
    # nothing to do is not an error
    assert lib.wan_flash_self_attn(ok, ok, ok, ok, 0, 24, 16, 16, 128, 0.1, 0, None) == 0


def test_workspace_sizes(W):
    lib = W._native.lib()
    B, H, L = 2, 24, 7854
    ws = lib.wan_self_attn_fused_workspace(B, H, L)
    assert ws >= B * L * 4 + B * L * H * 128 * 2 and ws % 256 == 0
    assert lib.wan_cross_attn_fused_workspace(B, H, L) >= B * L * 4
    assert lib.wan_self_attn_fused_workspace(0, H, L) == 0


def test_ops_fail_loudly_on_host_tensors(W):
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        W.ops.flash_self_attn(q, q, q, 0.1, 0)
    with pytest.raises(ValueError, match="CUDA"):
        W.ops.cross_attn(q, q, q, None, 0.1)


def test_ops_validate_layout(W):
    q = torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="head_dim"):
        W.ops.flash_self_attn(q, q, q, 0.1, 0)
    q = torch.zeros(1, 8, 2, 128, dtype=torch.float32)
    with pytest.raises(ValueError, match="bfloat16"):
        W.ops.flash_self_attn(q, q, q, 0.1, 0)


def test_custom_ops_have_fake_kernels(W):
    """torch.compile can trace the ops without running them (meta tensors)."""
    q = torch.empty(2, 100, 4, 128, dtype=torch.bfloat16, device="meta")
    out = torch.ops.wan_hip.flash_self_attn(q, q, q, 0.1, 0)
    assert out.shape == q.shape and out.device.type == "meta"
    out = torch.ops.wan_hip.cross_attn(q, q[:, :7], q[:, :7], None, 0.1)
    assert out.shape == q.shape


def test_adaln_validation_without_launching(W):
    N = W._native
    lib = N.lib()
    P = 256  # an aligned non-NULL stand-in pointer: every call below fails before any launch
    # dim not a multiple of 8 / too large
    assert lib.wan_adaln(P, None, None, P, 1, 4, 12, None, 1, -1, -1, -1, None, None, 1e-6, None) == 2
    assert lib.wan_adaln(P, None, None, P, 1, 4, 8200, None, 1, -1, -1, -1, None, None, 1e-6, None) == 2
    # seqlen not a multiple of frames
    rc = lib.wan_adaln(P, None, None, P, 1, 10, 64, P, 3, -1, 0, 1, None, None, 1e-6, None)
    assert rc == 1 and "frames" in N.last_error()
    # shift without scale, row index out of range
    assert lib.wan_adaln(P, None, None, P, 1, 4, 64, P, 1, -1, 0, -1, None, None, 1e-6, None) == 1
    assert lib.wan_adaln(P, P, P, P, 1, 4, 64, P, 1, 6, -1, -1, None, None, 1e-6, None) == 1
    # gate without y; modulation rows without e; weight without bias; misaligned
    assert lib.wan_adaln(P, None, None, P, 1, 4, 64, P, 1, 2, -1, -1, None, None, 1e-6, None) == 1
    assert lib.wan_adaln(P, None, None, P, 1, 4, 64, None, 1, -1, 0, 1, None, None, 1e-6, None) == 1
    assert lib.wan_adaln(P, None, None, P, 1, 4, 64, None, 1, -1, -1, -1, P, None, 1e-6, None) == 1
    rc = lib.wan_adaln(P + 2, None, None, P, 1, 4, 64, None, 1, -1, -1, -1, None, None, 1e-6, None)
    assert rc == 1 and "aligned" in N.last_error()
    # modulation without an output row
    assert lib.wan_adaln(P, P, P, None, 1, 4, 64, P, 1, -1, 0, 1, None, None, 1e-6, None) == 1
    # nothing to do is not an error
    assert lib.wan_adaln(P, None, None, P, 0, 4, 64, None, 1, -1, -1, -1, None, None, 1e-6, None) == 0
    # wan_adaln_ex: a second row set of 1..6 rows per frame, shift/scale indices within it,
    # the gate still indexing e's six rows
    ex = lib.wan_adaln_ex
    for rows in (0, 7):
        rc = ex(P, P, P, P, 1, 4, 64, P, 1, 5, P, rows, 0, 1, None, None, 1e-6, None)
        assert rc == 1 and "mod_rows" in N.last_error()
    rc = ex(P, P, P, P, 1, 4, 64, P, 1, 5, P, 2, 2, 1, None, None, 1e-6, None)
    assert rc == 1 and "out of range" in N.last_error()
    assert ex(P, P, P, P, 1, 4, 64, P, 1, 6, P, 2, 0, 1, None, None, 1e-6, None) == 1
    assert ex(P, P, P, P, 1, 4, 64, P, 1, 5, P + 4, 2, 0, 1, None, None, 1e-6, None) == 1
    # a NULL second row set is wan_adaln (six rows of e), so index 5 is in range there
    assert ex(P, P, P, P, 0, 4, 64, P, 1, 5, None, 0, 4, 5, None, None, 1e-6, None) == 0


def test_adaln_op_validates_on_cpu(W):
    x = torch.zeros(1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        W.ops.adaln(x)
    xm = torch.empty(2, 12, 64, dtype=torch.bfloat16, device="meta")
    r, h = torch.ops.wan_hip.adaln(xm, xm, None, 3, -1, -1, -1, None, None, 1e-6, True)
    assert r.shape == xm.shape and h.shape == xm.shape
    em = torch.empty(3, 2, 64, dtype=torch.bfloat16, device="meta")
    r, h = torch.ops.wan_hip.adaln(xm, xm, None, 3, -1, 0, 1, None, None, 1e-6, True, em)
    assert r.shape == xm.shape and h.shape == xm.shape


@pytest.mark.parametrize("scale", [0.0, -0.088, float("inf"), float("nan")])
def test_softmax_scale_must_be_finite_and_positive(W, scale):
    """The kernels fold softmax_scale * log2(e) into one FMA per score and take the running
    max over scaled scores: zero gives NaN on masked keys, a negative scale a wrong max.
    Every attention entry point rejects such a scale before any work."""
    N = W._native
    lib = N.lib()
    t = N.WanTensor(64, 24 * 128 * 16, 24 * 128, 128)
    p = 256
    calls = {
        "wan_flash_self_attn": lambda: lib.wan_flash_self_attn(t, t, t, t, 1, 24, 16, 16, 128, scale, 0, None),
        "wan_cross_attn": lambda: lib.wan_cross_attn(t, t, t, t, 1, 24, 16, 16, 128, scale, None, None),
        "wan_flash_attn_qnorm": lambda: lib.wan_flash_attn_qnorm(t, t, t, t, 1, 24, 16, 16, 128, p, p, None,
                                                                 None, scale, None, None),
        "wan_self_attn_fused": lambda: lib.wan_self_attn_fused(t, t, t, t, 1, 24, 16, 128, p, p, 1e-6, p, p,
                                                               scale, p, 1 << 30, None),
        "wan_cross_attn_fused": lambda: lib.wan_cross_attn_fused(t, t, t, t, 1, 24, 16, 16, 128, p, 1e-6, scale,
                                                                 None, p, 1 << 30, None),
    }
    for name, call in calls.items():
        assert call() == 2, name
        assert "softmax_scale" in N.last_error() and name in N.last_error()


def test_noalloc_rejects_rows_beyond_its_scratch(W):
    """wan_cross_attn_fused_noalloc's static scratch holds WAN_NOALLOC_MAX_ROWS query rows;
    a larger batch * seqlen_q is refused before any device call."""
    N = W._native
    lib = N.lib()
    t = N.WanTensor(64, 24 * 128 * 16, 24 * 128, 128)
    rc = lib.wan_cross_attn_fused_noalloc(t, t, t, t, 16, 24, 8193, 16, 128, 256, 1e-6, 0.088, None, None)
    assert rc == 2 and "static scratch" in N.last_error()
    rc = lib.wan_cross_attn_fused_noalloc(t, t, t, t, 1, 24, 16, 16, 128, 256, 1e-6, 0.0, None, None)
    assert rc == 2 and "softmax_scale" in N.last_error()


def test_qkv_gemm_and_sumsq_prep_validation_without_launching(W):
    """wan_qkv_proj_sumsq and wan_rms_norm_qk_sumsq refuse unsupported shapes, strides and
    missing operands before any device call."""
    N = W._native
    lib = N.lib()
    P = 256   # a 16-byte aligned stand-in address: nothing is launched
    gemm = lib.wan_qkv_proj_sumsq
    # N not a multiple of 256, K not a multiple of 64
    assert gemm(P, P, P, P, P, 64, 384, 128, 128, 128, 384, 128, None) == 2 and "multiple of 256" in N.last_error()
    assert gemm(P, P, P, P, P, 64, 512, 96, 96, 96, 512, 128, None) == 2 and "multiple" in N.last_error()
    # sq_cols beyond N or not a multiple of 64
    assert gemm(P, P, P, P, P, 64, 512, 128, 128, 128, 512, 576, None) == 1 and "sq_cols" in N.last_error()
    assert gemm(P, P, P, P, P, 64, 512, 128, 128, 128, 512, 96, None) == 1 and "sq_cols" in N.last_error()
    # row strides shorter than the rows, or not multiples of 8 elements
    assert gemm(P, P, P, P, P, 64, 512, 128, 64, 128, 512, 128, None) == 1 and "strides" in N.last_error()
    assert gemm(P, P, P, P, P, 64, 512, 128, 132, 128, 512, 128, None) == 1 and "strides" in N.last_error()
    # strides beyond the 32-bit tile offsets
    assert gemm(P, P, P, P, P, 64, 512, 128, 1 << 23, 128, 512, 128, None) == 2
    # a missing bias, misaligned output
    assert gemm(P, P, None, P, P, 64, 512, 128, 128, 128, 512, 128, None) == 1 and "NULL" in N.last_error()
    assert gemm(P, P, P, P + 2, P, 64, 512, 128, 128, 128, 512, 128, None) == 1
    # NULL x / w / out are refused whether or not sums of squares are asked for: with
    # sumsq NULL and sq_cols 0 only sumsq may be missing
    for args in ((None, P, P, P), (P, None, P, P), (P, P, P, None), (P, P, None, P)):
        assert gemm(*args, None, 64, 512, 128, 128, 128, 512, 0, None) == 1 and "NULL" in N.last_error()
    assert gemm(P, P, P, P, None, 64, 512, 128, 128, 128, 512, 128, None) == 1 and "sumsq" in N.last_error()
    # every pointer may be NULL when there are no rows
    assert gemm(None, None, None, None, None, 0, 512, 128, 128, 128, 512, 0, None) == 0
    # K = 0 is refused (no tile to accumulate); M = 0 is nothing to do
    assert gemm(P, P, P, P, P, 64, 512, 0, 128, 128, 512, 128, None) == 1 and "bad sizes" in N.last_error()
    assert gemm(P, P, P, P, P, 0, 512, 128, 128, 128, 512, 128, None) == 0

    t = N.WanTensor(64, 24 * 128 * 16, 24 * 128, 128)
    prep = lib.wan_rms_norm_qk_sumsq
    assert prep(t, P, 1, 16, 24, 128, P, 1e-6, P, P, None, P, None) == 1 and "required" in N.last_error()
    assert prep(t, P, 1, 16, 24, 128, P, 1e-6, P, P, P + 4, P, None) == 1 and "aligned" in N.last_error()
    assert prep(t, P, 1, 16, 40, 128, P, 1e-6, P, P, P, P, None) == 2 and "partial sums" in N.last_error()
    assert prep(t, P, 1, 16, 24, 64, P, 1e-6, P, P, P, P, None) == 2 and "head_dim" in N.last_error()
    assert prep(t, P, 0, 16, 24, 128, P, 1e-6, P, P, P, P, None) == 0
