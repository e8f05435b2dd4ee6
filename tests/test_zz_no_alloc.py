"""GPU: wan_cross_attn_fused_noalloc, the entry point that allocates nothing (its scratch
is a static array of the library), against wan_cross_attn_fused with a caller workspace.
Both run the same kernels, so the outputs must be the same bits.  Two calls in a row, the
second smaller, so the second runs on scratch that still holds the first call's rows;
each output is also checked against the oracle."""
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
D = 128
SCALE = D ** -0.5


def _case(W, B, H, Lq, Lk, lens, seed):
    N, lib = W._native, W._native.lib()
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b_, l_, H, D, generator=g).bfloat16()
               for b_, l_ in ((B, Lq), (B, Lk), (B, Lk)))
    gq = (1 + torch.rand(H * D, generator=g)).bfloat16()
    qd, kd, vd, gd = (t.to(DEV) for t in (q, k, v, gq))
    sk = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o_ws = torch.full_like(qd, float("nan"))
    o_na = torch.full_like(qd, float("nan"))
    need = lib.wan_cross_attn_fused_workspace(B, H, Lq)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    with torch.cuda.device(DEV):
        N.check("wan_cross_attn_fused", lib.wan_cross_attn_fused(
            N.tensor4(qd), N.tensor4(kd), N.tensor4(vd), N.tensor4(o_ws), B, H, Lq, Lk, D,
            gd.data_ptr(), 1e-6, SCALE, sk.data_ptr(), ws.data_ptr(), need, s))
        N.check("wan_cross_attn_fused_noalloc", lib.wan_cross_attn_fused_noalloc(
            N.tensor4(qd), N.tensor4(kd), N.tensor4(vd), N.tensor4(o_na), B, H, Lq, Lk, D,
            gd.data_ptr(), 1e-6, SCALE, sk.data_ptr(), s))
    torch.cuda.synchronize()
    qn = ref.rms(q.reshape(B, Lq, H * D), gq).view(B, Lq, H, D)
    want = ref.sdpa(qn.float(), k.float(), v.float(), seqlen_k=lens)
    return o_ws.cpu(), o_na.cpu(), want


def test_noalloc_matches_workspace_entry_point(W):
    cases = [(2, 24, 7854, 512, [470, 123], 1),     # config B
             (2, 3, 333, 77, [77, 5], 2)]            # smaller, on the same scratch
    for B, H, Lq, Lk, lens, seed in cases:
        print(f"noalloc case B={B} H={H} Lq={Lq} Lk={Lk} lens={lens}", flush=True)
        a, b, want = _case(W, B, H, Lq, Lk, lens, seed)
        assert torch.isfinite(b.float()).all()
        assert torch.equal(a, b)
        e = ref.rel_rms(b, want)
        print(f"  bit-identical to wan_cross_attn_fused; rel_rms vs fp32 oracle {e:.3e}", flush=True)
        assert e <= 5e-3
