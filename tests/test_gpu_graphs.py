"""GPU: the attention entry points captured in a HIP graph (torch.cuda.CUDAGraph) and
replayed.  Nothing on the path allocates device memory itself, synchronises or issues a
memset, so the calls can be recorded as they are: the fused self-attention (the K pass and
the attention kernel with the Q norm + RoPE), the fused cross-attention with per-sample key
lengths (the persistent kernel, which reads the lengths on the device) and the entry point
that allocates nothing go into one graph.  The graph is replayed three times, each time
after new values (and new key lengths) were copied into its inputs and the same calls ran
eagerly on them, with unrelated eager work in between: every replay must give the eager
bits."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
D = 128
SCALE = D ** -0.5


def test_graph_replays_match_eager(W):
    N, lib = W._native, W._native.lib()
    B, H, Lk = 2, 8, 77
    grid = (3, 6, 8)
    L = grid[0] * grid[1] * grid[2]
    cos, sin = (t.to(DEV) for t in W.rope.rope_tables(W.rope.wan_freqs(D), grid, D))

    def rnd(shape, seed, std=1.0):
        g = torch.Generator().manual_seed(seed)
        return (torch.randn(shape, generator=g) * std).bfloat16().to(DEV)

    q, k, v = rnd((B, L, H, D), 1), rnd((B, L, H, D), 2), rnd((B, L, H, D), 3)
    ck, cv = rnd((B, Lk, H, D), 4), rnd((B, Lk, H, D), 5)
    gq = (1 + rnd((H * D,), 6).float().abs()).bfloat16()
    gk = (1 + rnd((H * D,), 7).float().abs()).bfloat16()
    sk = torch.tensor([Lk, 30], dtype=torch.int32, device=DEV)
    out_na = torch.empty_like(q)

    def run():
        y_self = W.ops.self_attn_fused(q, k, v, gq, gk, 1e-6, cos, sin, SCALE)
        y_cross = W.ops.cross_attn_fused(q, ck, cv, gq, 1e-6, sk, SCALE)
        N.check("wan_cross_attn_fused_noalloc", lib.wan_cross_attn_fused_noalloc(
            N.tensor4(q), N.tensor4(ck), N.tensor4(cv), N.tensor4(out_na), B, H, L, Lk, D,
            gq.data_ptr(), 1e-6, SCALE, sk.data_ptr(), torch.cuda.current_stream().cuda_stream))
        return y_self, y_cross

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_self, g_cross = run()
    torch.cuda.synchronize()

    for r, lens in enumerate(([Lk, 30], [5, Lk], [0, 64])):
        print(f"replay {r}: key lengths {lens}", flush=True)
        for t, seed in ((q, 10), (k, 11), (v, 12), (ck, 13), (cv, 14)):
            t.copy_(rnd(t.shape, 100 * r + seed))
        sk.copy_(torch.tensor(lens, dtype=torch.int32))
        torch.cuda.synchronize()
        e_self, e_cross = run()
        e_na = out_na.clone()
        x = torch.randn(512, 512, device=DEV)
        (x @ x).sum().item()
        out_na.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(g_self.float()).all() and torch.isfinite(g_cross.float()).all()
        assert torch.equal(g_self, e_self)
        assert torch.equal(g_cross, e_cross)
        assert torch.equal(out_na, e_na) and torch.equal(out_na, e_cross)
