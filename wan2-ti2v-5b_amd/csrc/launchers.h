// Launchers of the kernels around the attention (prep.hip, adaln.hip, gemm.hip): their
// argument blocks and entry points (internal, C++ linkage), called by capi.hip.
#pragma once

#include "common.h"

namespace wan {

struct PrepArgs {
  Tensor4 x;            // input rows [B, L, H, 128]
  int B, L, H;
  float eps;
  float* inv_rms;       // out [B*L] fp32 (may be null)
  const bf16* gamma;    // [H*128] (null: no normalisation applied to `out`)
  const float* cos;     // [L, 64] fp32 (null: no rotation)
  const float* sin;
  bf16* out;            // out [B, L, H, 128] contiguous (null: statistics only)
  // Sums of squares given by the projection GEMM instead of computed from x:
  // partials sumsq[(sumsq_first + p) * B * L + token], p < sumsq_parts (null: from x).
  const float* sumsq;
  int sumsq_first, sumsq_parts;
};
int launch_rms_prep(const PrepArgs& a, hipStream_t s);
// Two tasks with the same H in one launch.
int launch_rms_prep2(const PrepArgs& a0, const PrepArgs& a1, hipStream_t s);

struct RopeArgs {
  Tensor4 x;
  int B, L, H;
  const float* cos;     // [L, 64]
  const float* sin;
  bf16* out;            // [B, L, H, 128] contiguous
};
int launch_rope(const RopeArgs& a, hipStream_t s);

// One adaLN stage of a block: residual update, LayerNorm, per-frame modulation.
struct AdaLNArgs {
  const bf16* x;        // [B, L, C] residual stream
  const bf16* y;        // [B, L, C] branch output added to x (null: none)
  bf16* x_out;          // [B, L, C] updated residual (null: not written)
  bf16* h_out;          // [B, L, C] normalised (and modulated) row (null: no LayerNorm)
  int B, L, C, F;       // F frames of L / F contiguous tokens each
  const bf16* e;        // [F, 6, C] modulation rows (block modulation + time projection)
  int gate_idx;         // row of e gating y (-1: ungated)
  const bf16* e_mod;    // [F, mod_rows, C] rows of the shift and scale (another block's, or
  int mod_rows;         // the output head's); e with 6 rows when the stage uses its own
  int shift_idx;        // rows of e_mod for the modulation (-1: none)
  int scale_idx;
  const bf16* ln_w;     // [C] LayerNorm affine weight / bias (null: not affine)
  const bf16* ln_b;
  float eps;
};
int launch_adaln(const AdaLNArgs& a, hipStream_t s);

// out = bf16(x w^T + bias) with per-head sums of squares of the first sq_cols columns.
struct GemmArgs {
  const bf16* x;        // [M, K] (row stride ldx)
  const bf16* w;        // [N, K] (row stride ldw), an nn.Linear weight
  const bf16* bias;     // [N]
  bf16* out;            // [M, N] (row stride ldo)
  float* sumsq;         // [sq_cols / 64, M]: per 64 columns, sum of bf16(out)^2
  int M, N, K;
  int64_t ldx, ldw, ldo;
  int sq_cols;          // multiple of 64, <= N
};
int launch_gemm_rowsq(const GemmArgs& a, hipStream_t s);

}  // namespace wan
