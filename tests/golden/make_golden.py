"""Writes tests/golden/attn_golden.npz: small known-answer vectors for the attention path.

The expected outputs are computed here in float64 numpy, independently of
oracle/ref.py (which is torch): the RMSNorm, the 3D-RoPE angle grid and
rotation, and the masked softmax attention are written out from their closed
forms.  Inputs are bf16-representable values (stored as float32) so that every
implementation starts from identical numbers.

Formulas (reference files the arithmetic follows):
  RMSNorm     x * (mean_c x^2 + eps)^-1/2 * gamma           models/fast_dit.py:134-147
  angles      theta_axis[p, j] = p * 10000^(-2j / D_axis), D_axis = 44/42/42 for
              frame/height/width; token (t, y, x) -> index t*h*w + y*w + x
                                                            wan/modules/rope_neuron.py:14-24,
                                                            models/fast_dit.py:548-558
  rotation    (x_2j, x_2j+1) -> (x_2j cos - x_2j+1 sin, x_2j sin + x_2j+1 cos)
                                                            models/fast_dit.py:163-169
  attention   softmax over keys j < len_b of q.k_j / sqrt(128), weighted sum of v_j
                                                            kernels/self_attention_nst.py:73-78

Run:  python tests/golden/make_golden.py   (deterministic; re-running rewrites the same file)
"""
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attn_golden.npz")
D = 128
EPS = 1e-6


def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bf16 (ties to even), returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def angles(grid):
    f, h, w = grid
    c = D // 2
    dims = [2 * (c - 2 * (c // 3)), 2 * (c // 3), 2 * (c // 3)]  # 44, 42, 42
    tabs = []
    for n, dim in zip((f, h, w), dims):
        j = np.arange(dim // 2, dtype=np.float64)
        tabs.append(np.outer(np.arange(n, dtype=np.float64), 10000.0 ** (-2.0 * j / dim)))
    ang = np.zeros((f, h, w, c))
    for t in range(f):
        for y in range(h):
            for x in range(w):
                ang[t, y, x] = np.concatenate([tabs[0][t], tabs[1][y], tabs[2][x]])
    return ang.reshape(f * h * w, c)


def rmsnorm(x, g):  # x [B, L, C]
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + EPS) * g


def rotate(x, ang):  # x [B, L, n, D]
    c, s = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]
    xr, xi = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = xr * c - xi * s
    out[..., 1::2] = xr * s + xi * c
    return out


def attend(q, k, v, lens):
    B, Lq, n, d = q.shape
    out = np.zeros((B, Lq, n, d))
    for b in range(B):
        m = lens[b]
        for h in range(n):
            s = q[b, :, h] @ k[b, :m, h].T / np.sqrt(d)
            p = np.exp(s - s.max(1, keepdims=True))
            out[b, :, h] = (p / p.sum(1, keepdims=True)) @ v[b, :m, h]
    return out


def main():
    rng = np.random.default_rng(20261201)
    arr = {}

    # fused self-attention: B=2, grid 2x3x5 (L=30), H=3
    grid = (2, 3, 5)
    B, H, L = 2, 3, 30
    q, k, v = (to_bf16(rng.standard_normal((B, L, H, D)).astype(np.float32)) for _ in range(3))
    gq = to_bf16((1 + 0.5 * rng.random(H * D)).astype(np.float32))
    gk = to_bf16((1 + 0.5 * rng.random(H * D)).astype(np.float32))
    ang = angles(grid)
    qn = rmsnorm(q.reshape(B, L, H * D).astype(np.float64), gq).reshape(B, L, H, D)
    kn = rmsnorm(k.reshape(B, L, H * D).astype(np.float64), gk).reshape(B, L, H, D)
    qr, kr = rotate(qn, ang), rotate(kn, ang)
    arr.update(self_q=q, self_k=k, self_v=v, self_gq=gq, self_gk=gk,
               self_grid=np.array(grid), self_angles=ang,
               self_qhat=qr, self_khat=kr,
               self_out=attend(qr, kr, v.astype(np.float64), [L] * B))

    # masked cross-attention with Q-RMSNorm: B=2, Lq=37, Lk=24, lens (5, 24), H=2
    B, H, Lq, Lk = 2, 2, 37, 24
    lens = np.array([5, 24], dtype=np.int32)
    q = to_bf16(rng.standard_normal((B, Lq, H, D)).astype(np.float32))
    ck, cv = (to_bf16(rng.standard_normal((B, Lk, H, D)).astype(np.float32)) for _ in range(2))
    gq = to_bf16((0.5 + rng.random(H * D)).astype(np.float32))
    qn = rmsnorm(q.reshape(B, Lq, H * D).astype(np.float64), gq).reshape(B, Lq, H, D)
    arr.update(cross_q=q, cross_k=ck, cross_v=cv, cross_gq=gq, cross_lens=lens,
               cross_out=attend(qn, ck.astype(np.float64), cv.astype(np.float64), lens))

    # plain attention with a key length below Lk (actual_seqlen_k): Lq=Lk=70, len 45, H=2, B=1
    q, k, v = (to_bf16(rng.standard_normal((1, 70, 2, D)).astype(np.float32)) for _ in range(3))
    arr.update(plain_q=q, plain_k=k, plain_v=v, plain_len=np.array(45),
               plain_out=attend(q.astype(np.float64), k.astype(np.float64),
                                v.astype(np.float64), [45]))

    np.savez_compressed(OUT, **{k: (v.astype(np.float32) if v.dtype == np.float64 else v)
                                for k, v in arr.items()})
    print(f"wrote {OUT}: {sorted(arr)}")


if __name__ == "__main__":
    main()
