// Shared types and helpers for the Wan DiT attention kernels (gfx950).
//
// Tensors cross the C-ABI as bf16 device pointers plus element strides in the
// [batch, token, head, channel] order of the DiT's q/k/v projections; the
// channel (head_dim) axis is always contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wan {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;    // Wan2.2-TI2V-5B: dim 3072 / 24 heads
constexpr int kRopePairs = 64;   // head_dim / 2 rotation pairs per head
constexpr int kNumXcd = 8;       // MI355X: 8 XCDs, each with its own L2

// A [batch, token, head, 128] bf16 view.
struct Tensor4 {
  const bf16* ptr;
  int64_t sb, st, sh;  // element strides of batch, token, head
};

// Records a message for wan_attn_last_error(); returns `code`.
int set_error(int code, const char* fmt, ...);

// Workgroup ids are dispatched round-robin over the XCDs (id % 8).  Remap so
// that each XCD receives one contiguous range of logical ids: neighbouring
// query blocks of the same head then share that XCD's L2 for K/V.
__device__ __forceinline__ int xcd_remap(int id, int n) {
  const int per = n / kNumXcd, rem = n % kNumXcd;
  const int xcd = id % kNumXcd, local = id / kNumXcd;
  return xcd < rem ? xcd * (per + 1) + local
                   : rem * (per + 1) + (xcd - rem) * per + local;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

}  // namespace wan

// Launchers implemented in the .hip translation units (internal, C++ linkage).
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
  int shift_idx;        // rows of e for the modulation (-1: none)
  int scale_idx;
  const bf16* ln_w;     // [C] LayerNorm affine weight / bias (null: not affine)
  const bf16* ln_b;
  float eps;
};
int launch_adaln(const AdaLNArgs& a, hipStream_t s);

enum QPrep { kQPlain = 0, kQNorm = 1, kQNormRope = 2 };

struct FlashArgs {
  Tensor4 q, k, v;
  bf16* o;
  int64_t o_sb, o_st, o_sh;
  int B, H, Lq, Lk;
  const int32_t* seqlen_k;  // device [B] per-sample key lengths, or null
  int seqlen_all;           // key length for every sample when seqlen_k is null
  float scale;              // softmax scale (1/sqrt(128) by default)
  int qprep;                // QPrep
  const float* inv_rms_q;   // [B*Lq] (kQNorm, kQNormRope)
  const bf16* gamma_q;      // [H*128]
  const float* cos;         // [Lq, 64] (kQNormRope)
  const float* sin;
};
int launch_flash_fwd(const FlashArgs& a, hipStream_t s);
// CU count of the current device (cached per device after the first query).
int device_cu_count();

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
