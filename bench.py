#!/usr/bin/env python
"""Benchmark of the Wan DiT self-attention hot path on one MI355X.

Workload (one step): the fused self-attention span of a Wan2.2-TI2V-5B block at
704x544x81 — B=2 (cond + uncond), L=7854 tokens (latent grid 21x17x22), 24
heads, head_dim 128, bf16 — i.e. QK-RMSNorm (eps 1e-6, over all 3072
channels) and 3D RoPE (44/42/42 split, theta 10000) fused into the flash
attention, on seeded N(0,1) projections already resident in HBM.

  value       whole-step TFLOP/s = 4*B*H*L^2*128 / step time (prep kernels included)
  roofline    the attention kernel alone: algorithmic FLOPs / its average launch
              time (HIP events around its launch on the stream it runs on), against
              MI355X dense bf16 MFMA peak (2.5 PFLOP/s)
  cpu_baseline  the reference's SDPA path (restated by the oracle: QK-RMSNorm + RoPE +
              torch SDPA) on the host cores over the whole config C workload in fp32,
              median of up to 3 runs; configs A and B and bf16 under "table"
  extra       the same path at L=1080 and the masked cross-attention (Lq=7854,
              512 text keys, per-sample lengths [470, 123]), with HBM GB/s; torch's
              own flash SDPA on the config C shapes, for comparison; the q/k/v
              projection + QK-RMSNorm prep by hipBLASLt and by the sums-of-squares GEMM; one
              WanAttentionBlock (D) and the 30-layer DiT, 10 UniPC steps (E):
              dit_s_per_step is the second half of the metric; the same DiT at the
              368x480x21 size (1080 tokens) as dit_E_L1080

Prints one JSON line on stdout.  Usage:
  python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S] [--no-cpu-baseline]
  python bench.py --profile-config {A,B,C,D,QKV,QKVGEMM} [--steps K]   (one config's steps only, for rocprofv3)
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

B, H, D = 2, 24, 128
GRID_C = (21, 17, 22)   # 704x544x81 -> latent 21 x 34 x 44 -> patch (1,2,2)
GRID_A = (6, 12, 15)    # 368x480x21 class of shapes: L=1080
L_TEXT = 512
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join("profiles", "flash_fwd_selfattn_L7854.md")
KERNEL_SOURCES = [os.path.join("wan2-ti2v-5b_amd", "csrc", f) for f in ("common.h", "flash_fwd.hip")]


def kernel_source_hash():
    """sha256 over the attention kernel's sources (common.h, flash_fwd.hip)."""
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SOURCES:
        with open(os.path.join(ROOT, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def profiled_traffic():
    """HBM bytes per launch of the config C attention kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (calibrated against a plain copy), and a note.  The
    summary records the hash of the kernel sources it measured; when the sources differ
    the figure is stale and None is returned."""
    import re
    try:
        text = open(os.path.join(ROOT, TRAFFIC_PROFILE)).read()
    except OSError:
        return None, "no traffic profile"
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    hm = re.search(r"^kernel_source_sha256:\s*([0-9a-f]{64})", text, re.M)
    if not m:
        return None, "no traffic figure in " + TRAFFIC_PROFILE
    if not hm or hm.group(1) != kernel_source_hash():
        return None, ("stale: " + TRAFFIC_PROFILE + " measured other kernel sources "
                      "(kernel_source_sha256 differs)")
    return int(m.group(1)), TRAFFIC_PROFILE + " (FETCH_SIZE x2.0 + WRITE_SIZE x1.0, per launch)"


def attn_flops(b, h, lq, lk):
    return 4.0 * b * h * lq * lk * D


def make_inputs(torch, grid, seed, dev):
    from importlib import import_module
    W = import_module("wan2_ti2v_5b_amd")
    L = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, L, H * D, generator=g).to(torch.bfloat16).view(B, L, H, D) for _ in range(3))
    gq = (1 + torch.randn(H * D, generator=g).abs() * 1.5).to(torch.bfloat16)
    gk = (1 + torch.randn(H * D, generator=g).abs() * 1.5).to(torch.bfloat16)
    cos, sin = W.rope.rope_tables(W.rope.wan_freqs(D), grid, D)
    host = dict(q=q, k=k, v=v, gq=gq, gk=gk, cos=cos, sin=sin)
    return {n: t.to(dev) for n, t in host.items()}, host


class FusedSelf:
    """One step = wan_rms_norm_qk (q statistics + k norm/rope, one launch) + attention with
    the q norm/rope in the kernel; buffers allocated once, outside the timed region."""

    def __init__(self, torch, W, t):
        self.torch, self.N = torch, W._native
        self.lib = W._native.lib()
        self.t = t
        q = t["q"]
        self.Bn, self.L = q.shape[0], q.shape[1]
        self.out = torch.empty_like(q)
        self.inv = torch.empty(self.Bn * self.L, dtype=torch.float32, device=q.device)
        self.khat = torch.empty_like(t["k"])
        self.stream = torch.cuda.current_stream().cuda_stream

    def prep(self):
        t, N, lib = self.t, self.N, self.lib
        N.check("qk prep", lib.wan_rms_norm_qk(N.tensor4(t["q"]), N.tensor4(t["k"]), self.khat.data_ptr(),
                                               self.Bn, self.L, H, D, t["gk"].data_ptr(), 1e-6,
                                               t["cos"].data_ptr(), t["sin"].data_ptr(),
                                               self.inv.data_ptr(), self.stream))

    def attn(self):
        t, N, lib = self.t, self.N, self.lib
        N.check("attention", lib.wan_flash_attn_qnorm(
            N.tensor4(t["q"]), N.tensor4(self.khat), N.tensor4(t["v"]), N.tensor4(self.out),
            self.Bn, H, self.L, self.L, D, self.inv.data_ptr(), t["gq"].data_ptr(),
            t["cos"].data_ptr(), t["sin"].data_ptr(), D ** -0.5, None, self.stream))


SETTLE_SECONDS = 0.3


def set_settle(seconds):
    global SETTLE_SECONDS
    SETTLE_SECONDS = seconds


def settle(torch, step_fns, seconds=None):
    """Untimed repetitions of the step for about `seconds` of device time before the warm-up
    steps.  After idle the part raises its clocks over the first ~0.1 s of work, so a short
    warm-up alone (5 steps of 1.4 ms) leaves the first timed steps below the steady clock.
    Nothing here is part of the timed region or changes what a step does."""
    seconds = SETTLE_SECONDS if seconds is None else seconds
    if seconds <= 0:
        return
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n, spent = 1, 0.0
    while spent < seconds * 1e3:
        e0.record()
        for _ in range(n):
            for f in step_fns:
                f()
        e1.record()
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1)
        n = min(2 * n, 256)


def time_steps(torch, step_fns, steps, warmup):
    """Runs `steps` steps of the stage functions; returns (total ms, [ms per stage]).

    The total comes from a pass with events only before the first and after the last step;
    the per-stage times from a second pass with an event pair around every launch (an event
    between two kernels delays the second one's dispatch, which the first pass keeps out of
    the step time)."""
    settle(torch, step_fns)
    for _ in range(warmup):
        for f in step_fns:
            f()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        for f in step_fns:
            f()
    end.record()
    torch.cuda.synchronize()
    total = start.elapsed_time(end)
    n = len(step_fns)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(n + 1)] for _ in range(steps)]
    for s in range(steps):
        ev[s][0].record()
        for i, f in enumerate(step_fns):
            f()
            ev[s][i + 1].record()
    torch.cuda.synchronize()
    stage = [sum(ev[s][i].elapsed_time(ev[s][i + 1]) for s in range(steps)) / steps for i in range(n)]
    return total, stage


def time_alone(torch, fn, launches):
    """ms per launch of `fn` run `launches` times back to back between one pair of events.
    An event recorded between two kernels delays the second one's dispatch; for kernels of
    tens of microseconds the per-stage figures of time_steps carry that delay, which the
    profiler's kernel durations do not."""
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(launches):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / launches


def bench_cross(torch, W, dev, steps, warmup):
    """Config B: q [2, 7854, 24, 128] N(0,1) with its RMSNorm fused, keys and values built
    as the pipeline builds them (a [2, 512, 4096] N(0,1) text context through the DiT's text
    embedding, then one block's lin_k + RMSNorm and lin_v, random std-0.02 weights), and
    per-sample key lengths drawn from U{16..512}."""
    g = torch.Generator().manual_seed(7)
    Lq = GRID_C[0] * GRID_C[1] * GRID_C[2]
    q = torch.randn(B, Lq, H, D, generator=g).to(torch.bfloat16).to(dev)
    # two draws of K/V size that earlier versions used directly: kept, so that the seeded
    # lengths below stay [470, 123]
    torch.randn(2, B, L_TEXT, H, D, generator=g)
    ctx = torch.randn(B, L_TEXT, 4096, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(dev)
    m = W.model.random_model(W.model.WanConfig(), num_layers=1, device=dev, seed=7)
    with torch.no_grad():
        ck, cv = W.fast_dit.cross_kv(m.blocks[0], m.text_embedding(ctx), "hip")
    del m, ctx
    gq = (1 + torch.randn(H * D, generator=g).abs()).to(torch.bfloat16).to(dev)
    lens = torch.randint(16, L_TEXT + 1, (B,), generator=g, dtype=torch.int32)
    lens_d = lens.to(dev)
    N, lib = W._native, W._native.lib()
    out = torch.empty_like(q)
    inv = torch.empty(B * Lq, dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream().cuda_stream

    def prep():
        N.check("q stats", lib.wan_rms_norm(N.tensor4(q), None, B, Lq, H, D, None, 1e-6, None, None,
                                            inv.data_ptr(), s))

    def attn():
        N.check("cross", lib.wan_flash_attn_qnorm(N.tensor4(q), N.tensor4(ck), N.tensor4(cv), N.tensor4(out),
                                                  B, H, Lq, L_TEXT, D, inv.data_ptr(), gq.data_ptr(),
                                                  None, None, D ** -0.5, lens_d.data_ptr(), s))
    total, (t_prep_step, t_attn_step) = time_steps(torch, [prep, attn], steps, warmup)
    t_prep, t_attn = time_alone(torch, prep, steps), time_alone(torch, attn, steps)
    ssum = int(lens.sum())
    host = dict(q=q.cpu(), ck=ck.cpu(), cv=cv.cpu(), gq=gq.cpu(), lens=lens.tolist(),
                flops=4.0 * H * Lq * D * ssum,
                workload=f"cross-attn B=2 Lq={Lq} Lkv={L_TEXT} seqlen_k={lens.tolist()}")
    flops = 4.0 * H * Lq * D * ssum
    byts = 2 * (B * Lq * H * D * 2) + 2 * ssum * H * D * 2   # q read, o write, k+v rows read
    return {
        "workload": f"cross-attn B=2 Lq={Lq} Lkv={L_TEXT} H=24 d=128, seqlen_k={lens.tolist()}, "
                    "K/V from a [2, 512, 4096] N(0,1) context via text_embedding + lin_k/RMSNorm, lin_v",
        "ms_per_step": total / steps, "attn_kernel_ms": t_attn, "q_stats_ms": t_prep,
        "attn_kernel_ms_in_step": t_attn_step, "q_stats_ms_in_step": t_prep_step,
        "kernel_timing": "attn_kernel_ms / q_stats_ms: launches back to back between one event pair; "
                         "*_in_step: an event pair around each launch within the interleaved steps",
        "tflops_kernel": flops / (t_attn * 1e-3) / 1e12,
        "hbm_gbs_kernel": byts / (t_attn * 1e-3) / 1e9,
        "frac_hbm_peak": byts / (t_attn * 1e-3) / 1e9 / PEAK_HBM_GBS,
    }, host


def bench_qkv(torch, W, dev, steps, warmup):
    """The block's q/k/v projection and QK-RMSNorm prep at config C (x [2, 7854, 3072],
    concatenated weight [9216, 3072]) by the two routes: hipBLASLt's GEMM, then
    wan_rms_norm_qk (q statistics + k norm/rope from the rows); or wan_qkv_proj_sumsq, the
    gfx950 GEMM that emits the sums of squares, then wan_rms_norm_qk_sumsq (no q read)."""
    import torch.nn.functional as F
    N_, lib = W._native, W._native.lib()
    L = GRID_C[0] * GRID_C[1] * GRID_C[2]
    C = H * D
    g = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(B, L, C, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(3 * C, C, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(3 * C, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    gk = (1 + torch.rand(C, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in W.rope.rope_tables(W.rope.wan_freqs(D), GRID_C, D))
    qkv = torch.empty(B, L, 3 * C, device=dev, dtype=torch.bfloat16)
    ss = torch.empty(4 * H, B * L, device=dev, dtype=torch.float32)
    inv = torch.empty(B * L, device=dev, dtype=torch.float32)
    khat = torch.empty(B, L, H, D, device=dev, dtype=torch.bfloat16)
    s = torch.cuda.current_stream().cuda_stream
    q = qkv[..., :C].view(B, L, H, D)
    k = qkv[..., C:2 * C].view(B, L, H, D)

    def gemm_blas():
        F.linear(x, w, bias)         # as the block calls it

    def prep_rows():
        N_.check("qk prep", lib.wan_rms_norm_qk(N_.tensor4(q), N_.tensor4(k), khat.data_ptr(), B, L, H, D,
                                                gk.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(),
                                                inv.data_ptr(), s))

    def gemm_sumsq():
        N_.check("qkv gemm", lib.wan_qkv_proj_sumsq(x.data_ptr(), w.data_ptr(), bias.data_ptr(), qkv.data_ptr(),
                                                    ss.data_ptr(), B * L, 3 * C, C, C, C, 3 * C, 2 * C, s))

    def prep_sums():
        N_.check("qk prep from sums", lib.wan_rms_norm_qk_sumsq(N_.tensor4(k), khat.data_ptr(), B, L, H, D,
                                                                gk.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(),
                                                                ss.data_ptr(), inv.data_ptr(), s))
    # the two routes interleaved in the same steps (prep_rows reads the q/k the sums GEMM wrote)
    _, (t_gemm, t_sums, t_blas, t_rows) = time_steps(torch, [gemm_sumsq, prep_sums, gemm_blas, prep_rows],
                                                      steps, warmup)
    flops = 2.0 * B * L * 3 * C * C
    return {"qkv_projection": {
        "workload": f"x [2, {L}, 3072] x [9216, 3072]^T + bias, then the QK-RMSNorm prep of the fused self-attention",
        "hipblaslt_gemm_ms": t_blas, "prep_from_rows_ms": t_rows, "hipblaslt_route_ms": t_blas + t_rows,
        "sumsq_gemm_ms": t_gemm, "prep_from_sums_ms": t_sums, "sumsq_route_ms": t_gemm + t_sums,
        "hipblaslt_tflops": flops / (t_blas * 1e-3) / 1e12, "sumsq_gemm_tflops": flops / (t_gemm * 1e-3) / 1e12}}


def qkv_gemms_alone(torch, W, dev, launches):
    """The QKV projection GEMM with the sums of squares and hipBLASLt's F.linear on the same
    inputs, each `launches` times back to back with nothing in between (for counters that
    other kernels between the launches would disturb, such as the L2 misses)."""
    import torch.nn.functional as F
    N_, lib = W._native, W._native.lib()
    L = GRID_C[0] * GRID_C[1] * GRID_C[2]
    C = H * D
    g = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(B * L, C, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(3 * C, C, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(3 * C, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    out = torch.empty(B * L, 3 * C, device=dev, dtype=torch.bfloat16)
    ss = torch.empty(4 * H, B * L, device=dev, dtype=torch.float32)
    s = torch.cuda.current_stream().cuda_stream

    def gemm():
        N_.check("qkv gemm", lib.wan_qkv_proj_sumsq(x.data_ptr(), w.data_ptr(), bias.data_ptr(), out.data_ptr(),
                                                    ss.data_ptr(), B * L, 3 * C, C, C, C, 3 * C, 2 * C, s))
    res = {}
    for name, fn in (("sumsq_gemm_ms", gemm), ("hipblaslt_gemm_ms", lambda: F.linear(x, w, bias))):
        res[name] = time_alone(torch, fn, launches)
    return res


def bench_torch_sdpa(torch, t, steps, warmup):
    """torch's own F.scaled_dot_product_attention (flash backend) on the config C shapes:
    plain attention of the same q/k/v sizes (no norm, no rotation), for comparison."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    q, k, v = (t[n].transpose(1, 2).contiguous() for n in ("q", "k", "v"))
    L = q.shape[2]
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            total, (ms,) = time_steps(torch, [lambda: F.scaled_dot_product_attention(q, k, v)], steps, warmup)
    except RuntimeError as e:
        return {"torch_sdpa_L7854": {"error": str(e)[:200]}}
    return {"torch_sdpa_L7854": {
        "workload": f"torch F.scaled_dot_product_attention, flash backend, B=2 H=24 L={L} d=128 bf16",
        "ms": ms, "tflops": attn_flops(B, H, L, L) / (ms * 1e-3) / 1e12}}


def dit_setup(torch, W, dev, layers, grid=GRID_C, model=None):
    """A `layers`-layer DiT at the token grid `grid` (704x544x81 by default) with random bf16
    weights (std 0.02), the HIP attention path, both prompts' cross K/V set and one warm-up
    forward done.  `model`: reuse these weights instead of drawing new ones."""
    cfg = W.model.WanConfig()
    if model is None:
        model = W.model.random_model(cfg, num_layers=layers, device=dev, seed=0)
    fast = W.fast_dit.FastWanDiT(model, grid, cfg.sample_guide_scale, attn_impl="hip", cross_impl="hip")
    g = torch.Generator().manual_seed(5)
    f, h, w = grid
    latent = torch.randn(cfg.in_dim, f, 2 * h, 2 * w, generator=g).to(dev)     # [48, 21, 34, 44]
    ctx_c = torch.randn(1, cfg.text_len, cfg.text_dim, generator=g).to(dev)
    ctx_n = torch.randn(1, cfg.text_len, cfg.text_dim, generator=g).to(dev)
    image_latent = torch.randn(cfg.in_dim, 1, 2 * h, 2 * w, generator=g).to(dev)
    fast.set_context(ctx_c, ctx_n)
    fast(latent, torch.tensor(999))                          # warm-up (GEMM heuristics, allocator)
    torch.cuda.synchronize()
    return cfg, fast, latent, image_latent


def block_inputs(torch, fast, latent):
    """The first block and its inputs as the DiT gives them at t = 500."""
    _, e0 = fast.time_rows(torch.tensor(500))
    ck, cv = fast.context[0]
    return fast.blocks[0], (fast.patch(latent), e0, fast.cos, fast.sin, ck, cv)


def profile_block(torch, W, dev, steps):
    """Only `steps` forwards of one WanAttentionBlock at L=7854 (for rocprofv3)."""
    _, fast, latent, _ = dit_setup(torch, W, dev, 1)
    blk, inputs = block_inputs(torch, fast, latent)
    for _ in range(2):
        blk(*inputs)
    e_a, e_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e_a.record()
    for _ in range(steps):
        blk(*inputs)
    e_b.record()
    torch.cuda.synchronize()
    return e_a.elapsed_time(e_b) / steps


def bench_dit(torch, W, dev, steps, layers):
    """Config D (one WanAttentionBlock at L=7854) and config E (the 30-layer DiT, 10 UniPC
    steps at 704x544x81) with random bf16 weights (std 0.02) and the HIP attention path."""
    cfg = W.model.WanConfig()
    cfg, fast, latent, image_latent = dit_setup(torch, W, dev, layers, model=fast_model(cfg, W, dev, layers))

    # config D: one block, its inputs as in the DiT
    blk, inputs = block_inputs(torch, fast, latent)
    x = inputs[0]
    for _ in range(2):
        blk(*inputs)
    e_a, e_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e_a.record()
    for _ in range(5):
        y = blk(*inputs)
    e_b.record()
    torch.cuda.synchronize()
    block_ms = e_a.elapsed_time(e_b) / 5
    L = x.shape[1]
    C, Fd = cfg.dim, cfg.ffn_dim
    block_flops = 2.0 * B * L * (6 * C * C + 2 * C * Fd) + attn_flops(B, H, L, L) + 4.0 * B * H * L * L_TEXT * D
    del y

    # config E: the denoising loop
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_a.record()
    final = W.fast_dit.denoise(fast, latent, steps, cfg.sample_shift, image_latent=image_latent)
    e_b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dit_s = e_a.elapsed_time(e_b) / 1e3
    finite = bool(torch.isfinite(final.float()).all())
    step_flops = layers * block_flops
    res = {
        "block_D": {"workload": "one WanAttentionBlock forward, B=2, L=7854, dim 3072, ffn 14336, "
                                "24 heads, 512 text keys, random bf16 weights",
                    "ms": block_ms, "tflops": block_flops / (block_ms * 1e-3) / 1e12},
        "dit_E": {"workload": f"{layers}-layer Wan2.2-TI2V-5B DiT, {steps} UniPC steps (shift 5.0, guide 5.0), "
                              "704x544x81 (latent 48x21x34x44, L=7854), CFG batch 2, random bf16 weights",
                  "s_per_step": dit_s / steps, "wall_s_per_step": wall / steps,
                  "tflops": step_flops / (dit_s / steps) / 1e12, "finite": finite},
    }
    del final, fast

    # the same DiT at the reference's 368x480x21 size: generated at 384x480 (latent
    # 48 x 6 x 24 x 30, 1080 tokens) and centre-cropped, as README.md:41 of the reference
    _, fast_a, latent_a, image_a = dit_setup(torch, W, dev, layers, GRID_A, model=fast_model(cfg, W, dev, layers))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_a.record()
    final = W.fast_dit.denoise(fast_a, latent_a, steps, cfg.sample_shift, image_latent=image_a)
    e_b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    s_a = e_a.elapsed_time(e_b) / 1e3 / steps
    LA = GRID_A[0] * GRID_A[1] * GRID_A[2]
    flops_a = layers * (2.0 * B * LA * (6 * C * C + 2 * C * Fd) + attn_flops(B, H, LA, LA)
                        + 4.0 * B * H * LA * L_TEXT * D)
    res["dit_E_L1080"] = {
        "workload": f"{layers}-layer Wan2.2-TI2V-5B DiT, {steps} UniPC steps, 368x480x21 generated at 384x480 "
                    "(latent 48x6x24x30, L=1080), CFG batch 2, random bf16 weights (the same as dit_E)",
        "s_per_step": s_a, "wall_s_per_step": wall / steps, "tflops": flops_a / s_a / 1e12,
        "finite": bool(torch.isfinite(final.float()).all())}
    return res


_MODEL = {}


def fast_model(cfg, W, dev, layers):
    """The random-weight model of the DiT runs, drawn once per process."""
    if layers not in _MODEL:
        _MODEL[layers] = W.model.random_model(cfg, num_layers=layers, device=dev, seed=0)
    return _MODEL[layers]


def cpu_baseline(torch, hosts, seconds):
    """The reference's SDPA path (models/fast_dit.py:186-189, restated by the oracle) on the
    host cores, in fp32 and in bf16, for configs C, A and B on the GPU run's own inputs:
    QK-RMSNorm + RoPE + SDPA over every (batch, head) for the self-attention, Q-RMSNorm +
    masked SDPA for the cross-attention.  Each is the median of up to 3 repetitions (after
    one warm-up for A and B), within about `seconds` of CPU work in all; config C in fp32,
    the headline workload, always gets at least one.  Returns the headline object (config C,
    fp32) with the whole table under "table"."""
    sys.path.insert(0, ROOT)
    from oracle import ref
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)

    def self_path(h, dt):
        q, k, v = (h[n].to(dt) for n in "qkv")
        Bn, L, Hn, Dd = q.shape
        qn, kn = ref.rms_qk(q.reshape(Bn, L, Hn * Dd), k.reshape(Bn, L, Hn * Dd), h["gq"].to(dt), h["gk"].to(dt))
        return ref.sdpa(ref.rope(qn.view(Bn, L, Hn, Dd), h["cos"], h["sin"]),
                        ref.rope(kn.view(Bn, L, Hn, Dd), h["cos"], h["sin"]), v)

    def cross_path(h, dt):
        q, ck, cv = (h[n].to(dt) for n in ("q", "ck", "cv"))
        Bn, L, Hn, Dd = q.shape
        qn = ref.rms(q.reshape(Bn, L, Hn * Dd), h["gq"].to(dt)).view(Bn, L, Hn, Dd)
        return ref.sdpa(qn, ck, cv, seqlen_k=h["lens"])

    plan = [("C", torch.float32, 3), ("A", torch.float32, 3), ("B", torch.float32, 3),
            ("A", torch.bfloat16, 3), ("B", torch.bfloat16, 3), ("C", torch.bfloat16, 3)]
    table, spent = {}, 0.0
    for cfg, dt, reps in plan:
        h = hosts.get(cfg)
        if h is None:
            continue
        fn = cross_path if cfg == "B" else self_path
        if cfg != "C":
            fn(h, dt)
        times = []
        for r in range(reps):
            if spent >= seconds and not (cfg == "C" and dt == torch.float32 and r == 0):
                break
            t0 = time.perf_counter()
            fn(h, dt)
            times.append(time.perf_counter() - t0)
            spent += times[-1]
        if not times:
            continue
        med = sorted(times)[len(times) // 2]
        key = f"{cfg}_{'fp32' if dt == torch.float32 else 'bf16'}"
        table[key] = {"ms": med * 1e3, "tflops": h["flops"] / med / 1e12, "reps": len(times),
                      "workload": h["workload"]}
    c = table["C_fp32"]
    return {
        "value": c["tflops"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"the whole config C workload (B=2, L=7854, 24 heads: QK-RMSNorm + RoPE + fp32 "
                  f"torch SDPA, oracle/ref.py), median of {c['reps']} run(s), {c['ms'] / 1e3:.2f} s each; "
                  f"fp32 and bf16 for configs A, B, C under 'table'",
        "table": table,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # after idle the part raises its clocks over the first ~0.1 s of work: 100 untimed steps
    # (~0.15 s at config C) put the timed steps at the steady state
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--settle-seconds", type=float, default=SETTLE_SECONDS,
                    help="untimed clock settle before each timed config's warm-up steps (0: none)")
    ap.add_argument("--cpu-seconds", type=float, default=25.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-dit", action="store_true", help="skip the block (D) and 30-layer DiT (E) runs")
    ap.add_argument("--dit-steps", type=int, default=10)
    ap.add_argument("--dit-layers", type=int, default=30)
    ap.add_argument("--profile-config", choices=["A", "B", "C", "D", "QKV", "QKVGEMM"], default=None,
                    help="only run the timed steps of one attention config, of one block (D), or "
                         "of the two QKV projection routes (for rocprofv3)")
    ap.add_argument("--profile-copy", type=int, default=0, metavar="BYTES",
                    help="only run 10 device-to-device copies of BYTES (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the attention path runs all 24 heads and CFG batch 2 on "
              f"a single MI355X and has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    set_settle(args.settle_seconds)
    sys.path.insert(0, ROOT)
    import __graft_entry__
    W = __graft_entry__.load_package()
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile_copy:
        src = torch.ones(args.profile_copy // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {src.numel() * 4} bytes 10 times")
        return
    if args.profile_config:
        if args.profile_config == "B":
            r, _ = bench_cross(torch, W, dev, args.steps, args.warmup)
            log(f"config B: attention kernel {r['attn_kernel_ms']:.4f} ms")
        elif args.profile_config == "D":
            log(f"config D: {profile_block(torch, W, dev, args.steps):.3f} ms per block")
        elif args.profile_config == "QKVGEMM":
            log(f"QKV GEMMs alone: {json.dumps(qkv_gemms_alone(torch, W, dev, args.steps))}")
        elif args.profile_config == "QKV":
            r = bench_qkv(torch, W, dev, args.steps, args.warmup)["qkv_projection"]
            log(f"QKV projection: gemm {r['sumsq_gemm_ms']:.4f} ms, hipBLASLt {r['hipblaslt_gemm_ms']:.4f} ms")
        else:
            t, _ = make_inputs(torch, GRID_C if args.profile_config == "C" else GRID_A, 0, dev)
            fs = FusedSelf(torch, W, t)
            total, (_, t_attn) = time_steps(torch, [fs.prep, fs.attn], args.steps, args.warmup)
            log(f"config {args.profile_config}: attention kernel {t_attn:.4f} ms")
        return
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    t, host = make_inputs(torch, GRID_C, 0, dev)
    L = t["q"].shape[1]
    fs = FusedSelf(torch, W, t)
    total, (t_prep, t_attn) = time_steps(torch, [fs.prep, fs.attn], args.steps, args.warmup)
    ms = total / args.steps
    t_attn_alone = time_alone(torch, fs.attn, min(args.steps, 20))
    flops = attn_flops(B, H, L, L)
    achieved = flops / (t_attn * 1e-3) / 1e12
    log(f"config C: step {ms:.3f} ms (prep {t_prep:.3f} ms, attention kernel {t_attn:.3f} ms) "
        f"-> {flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s step, {achieved:.1f} TFLOP/s kernel")

    extra = {}
    if not args.no_extra:
        tA, hostA = make_inputs(torch, GRID_A, 1, dev)
        fA = FusedSelf(torch, W, tA)
        totA, (pA_step, aA_step) = time_steps(torch, [fA.prep, fA.attn], args.steps, args.warmup)
        pA, aA = time_alone(torch, fA.prep, args.steps), time_alone(torch, fA.attn, args.steps)
        LA = tA["q"].shape[1]
        extra["self_attn_L1080"] = {
            "workload": "fused self-attn B=2 L=1080 (grid 6x12x15) H=24 d=128",
            "ms_per_step": totA / args.steps, "attn_kernel_ms": aA, "prep_ms": pA,
            "attn_kernel_ms_in_step": aA_step, "prep_ms_in_step": pA_step,
            "kernel_timing": "attn_kernel_ms / prep_ms: launches back to back between one event pair; "
                             "*_in_step: an event pair around each launch within the interleaved steps",
            "tflops_step": attn_flops(B, H, LA, LA) / (totA / args.steps * 1e-3) / 1e12,
            "tflops_kernel": attn_flops(B, H, LA, LA) / (aA * 1e-3) / 1e12}
        extra["cross_attn"], hostB = bench_cross(torch, W, dev, args.steps, args.warmup)
        extra.update(bench_torch_sdpa(torch, t, min(args.steps, 20), 3))
        extra.update(bench_qkv(torch, W, dev, min(args.steps, 20), 3))
        log(f"extra: {json.dumps(extra)}")
    if not args.no_dit:
        extra.update(bench_dit(torch, W, dev, args.dit_steps, args.dit_layers))
        log(f"block D: {extra['block_D']['ms']:.2f} ms; DiT E: {extra['dit_E']['s_per_step']:.3f} s/step "
            f"(L=1080: {extra['dit_E_L1080']['s_per_step']:.4f} s/step)")

    cpu = None
    if not args.no_cpu_baseline:
        host["flops"] = flops
        host["workload"] = f"self-attn B=2 L={L} (grid 21x17x22)"
        hosts = {"C": host}
        if not args.no_extra:
            LA = hostA["q"].shape[1]
            hostA.update(flops=attn_flops(B, H, LA, LA), workload=f"self-attn B=2 L={LA} (grid 6x12x15)")
            hosts.update(A=hostA, B=hostB)
        else:
            hosts.update(A=None, B=None)
        cpu = cpu_baseline(torch, {k: v for k, v in hosts.items()}, args.cpu_seconds)
        log(f"cpu baseline: {json.dumps(cpu)}")

    traffic, traffic_note = profiled_traffic()
    line = {
        "metric": "self-attn TFLOP/s @L=7854 (% bf16 MFMA peak); DiT s/step 704x544x81",
        "value": flops / (ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v projections, peaky QK-norm gammas)",
        "config": {"workload": "fused QK-RMSNorm + 3D-RoPE + flash self-attention, B=2 (CFG), "
                               "L=7854 (latent 21x17x22, 704x544x81), 24 heads, head_dim 128",
                   "global_batch": B, "seq_len": L, "heads": H, "head_dim": D, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "flash_fwd_kernel<8,2> (attention with the Q RMSNorm + RoPE applied in-kernel)",
                     "bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "traffic_source": traffic_note, "kernel_source_sha256": kernel_source_hash(),
                     "kernel_ms": t_attn, "flops_per_launch": flops,
                     "kernel_ms_back_to_back": t_attn_alone},
        "cpu_baseline": cpu,
        "prep_ms": t_prep,
        "dit_s_per_step": extra.get("dit_E", {}).get("s_per_step"),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
