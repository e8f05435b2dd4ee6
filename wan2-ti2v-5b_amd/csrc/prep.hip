// Token-row kernels of the attention path: the QK-RMSNorm statistics (and the
// normalised, rotated K rows the attention kernel streams), and a standalone
// 3D-RoPE rotation.
//
// Rounding follows the reference's bf16 graph exactly:
//   _tp_rms_qk  models/fast_dit.py:134-147   t = bf16(x * rsqrt(sum(x^2)/C + eps)); u = bf16(t * gamma)
//   _rope       models/fast_dit.py:163-169   fp32 pair rotation of u, one bf16 rounding
// Contraction into FMAs is disabled in the rotation so each product and sum is
// rounded as the separate torch ops round it.
#include "launchers.h"

namespace wan {

namespace {

constexpr int kMaxChunksPerLane = 16;  // supports H*128 <= 8192 channels per token

// Rotate interleaved pairs of 8 consecutive channels d0..d0+7 of one token.
__device__ __forceinline__ void rope8(float u[8], const float* cos_row,
                                      const float* sin_row, int d0) {
#pragma clang fp contract(off)
  const f32x4 c = *reinterpret_cast<const f32x4*>(cos_row + d0 / 2);
  const f32x4 s = *reinterpret_cast<const f32x4*>(sin_row + d0 / 2);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float xr = u[2 * j], xi = u[2 * j + 1];
    const float a = xr * c[j];
    const float b = xi * s[j];
    const float e = xr * s[j];
    const float f = xi * c[j];
    u[2 * j] = a - b;
    u[2 * j + 1] = e + f;
  }
}

// One wave per token row: sum of squares over all H*128 channels, then
// optionally the normalised (and rotated) row.  NCH: 8-channel chunks per lane
// (H*16 <= 64*NCH), so the row's loads are issued unconditionally together.  The
// rows are read once here: non-temporal loads (4% faster alone at B=2, L=7854 than
// plain ones, ~2 us a launch, below what a whole block forward resolves; the written
// rows stay cacheable, the attention kernel reads them next).
template <int NCH>
__device__ __forceinline__ void rms_prep_rows(const PrepArgs& a, int block) {
  const int lane = threadIdx.x & 63;
  const int tok = block * 4 + (threadIdx.x >> 6);
  if (tok >= a.B * a.L) return;
  const int b = tok / a.L, l = tok - b * a.L;
  const int nchunks = a.H * 16;
  const bf16* row = a.x.ptr + b * a.x.sb + (int64_t)l * a.x.st;

  bf16x8 xv[NCH];
  float ss = 0.f;
  if (a.sumsq != nullptr) {
    // the projection GEMM's partial sums (one per lane, then the wave's sum); the row
    // itself is read only when the normalised row is wanted
    if (lane < a.sumsq_parts) ss = a.sumsq[(int64_t)(a.sumsq_first + lane) * (a.B * a.L) + tok];
    if (a.out != nullptr) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunks) xv[i] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(row + (c >> 4) * a.x.sh + (c & 15) * 8));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunks) {
        const int h = c >> 4, d0 = (c & 15) * 8;
        xv[i] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(row + h * a.x.sh + d0));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float f = (float)xv[i][j];
          ss += f * f;
        }
      }
    }
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)(a.H * kHeadDim) + a.eps);
  if (a.inv_rms != nullptr && lane == 0) a.inv_rms[tok] = inv;
  if (a.out == nullptr) return;

  const float* cos_row = a.cos ? a.cos + (int64_t)l * kRopePairs : nullptr;
  const float* sin_row = a.sin ? a.sin + (int64_t)l * kRopePairs : nullptr;
  bf16* orow = a.out + (int64_t)tok * a.H * kHeadDim;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) {
      const int h = c >> 4, d0 = (c & 15) * 8;
      const bf16x8 g = *reinterpret_cast<const bf16x8*>(a.gamma + h * kHeadDim + d0);
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bf16 t = (bf16)((float)xv[i][j] * inv);
        u[j] = (float)(bf16)((float)t * (float)g[j]);
      }
      if (cos_row) rope8(u, cos_row, sin_row, d0);
      bf16x8 r;
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = (bf16)u[j];
      *reinterpret_cast<bf16x8*>(orow + h * kHeadDim + d0) = r;
    }
  }
}

template <int NCH>
__global__ __launch_bounds__(256) void rms_prep_kernel(const PrepArgs a) {
  rms_prep_rows<NCH>(a, blockIdx.x);
}

// Two independent tasks (the q statistics and the k norm + rotation of one
// self-attention call) in one launch: blocks [0, blocks0) run a0, the rest a1.
template <int NCH>
__global__ __launch_bounds__(256) void rms_prep2_kernel(const PrepArgs a0, const PrepArgs a1, int blocks0) {
  if ((int)blockIdx.x < blocks0) rms_prep_rows<NCH>(a0, blockIdx.x);
  else rms_prep_rows<NCH>(a1, blockIdx.x - blocks0);
}


// One thread per 8 channels: out = rope(x), the _rope semantics on its own.
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a) {
  const int64_t chunk = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.L * a.H * 16;
  if (chunk >= total) return;
  const int d0 = (int)(chunk & 15) * 8;
  int64_t rest = chunk >> 4;
  const int h = (int)(rest % a.H);
  rest /= a.H;
  const int l = (int)(rest % a.L);
  const int b = (int)(rest / a.L);
  const bf16x8 x = *reinterpret_cast<const bf16x8*>(a.x.ptr + b * a.x.sb + (int64_t)l * a.x.st +
                                                    h * a.x.sh + d0);
  float u[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) u[j] = (float)x[j];
  rope8(u, a.cos + (int64_t)l * kRopePairs, a.sin + (int64_t)l * kRopePairs, d0);
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (bf16)u[j];
  *reinterpret_cast<bf16x8*>(a.out + chunk * 8) = r;
}

}  // namespace

int launch_rms_prep(const PrepArgs& a, hipStream_t s) {
  const int rows = a.B * a.L;
  if (rows == 0) return 0;
  const int nch = a.H * 16;
  if (nch > 64 * kMaxChunksPerLane) return set_error(2, "rms_prep: H*128=%d channels exceeds 8192", a.H * 128);
  const dim3 grid((rows + 3) / 4), block(256);
  if (nch <= 64) hipLaunchKernelGGL(rms_prep_kernel<1>, grid, block, 0, s, a);
  else if (nch <= 128) hipLaunchKernelGGL(rms_prep_kernel<2>, grid, block, 0, s, a);
  else if (nch <= 256) hipLaunchKernelGGL(rms_prep_kernel<4>, grid, block, 0, s, a);
  else if (nch <= 384) hipLaunchKernelGGL(rms_prep_kernel<6>, grid, block, 0, s, a);
  else if (nch <= 512) hipLaunchKernelGGL(rms_prep_kernel<8>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(rms_prep_kernel<16>, grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "rms_prep launch: %s", hipGetErrorString(e));
}

int launch_rms_prep2(const PrepArgs& a0, const PrepArgs& a1, hipStream_t s) {
  if (a0.H != a1.H) return set_error(1, "rms_prep: the paired tasks differ in heads");
  const int rows0 = a0.B * a0.L, rows1 = a1.B * a1.L;
  if (rows0 == 0) return launch_rms_prep(a1, s);
  if (rows1 == 0) return launch_rms_prep(a0, s);
  const int nch = a0.H * 16;
  if (nch > 64 * kMaxChunksPerLane) return set_error(2, "rms_prep: H*128=%d channels exceeds 8192", a0.H * 128);
  const int blocks0 = (rows0 + 3) / 4;
  const dim3 grid(blocks0 + (rows1 + 3) / 4), block(256);
  if (nch <= 64) hipLaunchKernelGGL(rms_prep2_kernel<1>, grid, block, 0, s, a0, a1, blocks0);
  else if (nch <= 128) hipLaunchKernelGGL(rms_prep2_kernel<2>, grid, block, 0, s, a0, a1, blocks0);
  else if (nch <= 256) hipLaunchKernelGGL(rms_prep2_kernel<4>, grid, block, 0, s, a0, a1, blocks0);
  else if (nch <= 384) hipLaunchKernelGGL(rms_prep2_kernel<6>, grid, block, 0, s, a0, a1, blocks0);
  else if (nch <= 512) hipLaunchKernelGGL(rms_prep2_kernel<8>, grid, block, 0, s, a0, a1, blocks0);
  else hipLaunchKernelGGL(rms_prep2_kernel<16>, grid, block, 0, s, a0, a1, blocks0);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "rms_prep launch: %s", hipGetErrorString(e));
}

int launch_rope(const RopeArgs& a, hipStream_t s) {
  const int64_t total = (int64_t)a.B * a.L * a.H * 16;
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "rope launch: %s", hipGetErrorString(e));
}

}  // namespace wan
