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

// The attention launcher (flash_fwd.hip; internal, C++ linkage).  The other kernels'
// launchers are declared in launchers.h, so that this header holds only what the
// attention kernels are compiled from.
namespace wan {

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

}  // namespace wan
