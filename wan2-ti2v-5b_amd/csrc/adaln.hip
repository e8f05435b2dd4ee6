// The pointwise chain around a WanAttentionBlock's GEMMs, fused into one pass
// per stage (adaLN: residual update, LayerNorm, per-frame modulation):
//
//   r = x                          (y absent)
//   r = bf16(x + y)                (y, no gate)
//   r = bf16(x + bf16(y * g[f]))   (y, gate row g = e[f, gate_idx])
//   ln = bf16(LayerNorm(r))        fp32 mean / biased variance over the dim channels,
//                                  [* w + b] when the norm is affine
//   h = ln                         (no modulation)
//   h = bf16(bf16(ln * bf16(1 + m[f, scale_idx])) + m[f, shift_idx])
//
// The modulation rows m are e itself, or another row set: the next block's rows when
// one pass ends a block (gated residual) and starts the next (norm1 + modulate), or
// the output head's two rows per frame after the last block.
//
// f is the frame of the token (tokens of one frame are contiguous).  The
// rounding points are those of the reference's eager bf16 graph:
//   _modulate / _gate      models/fast_dit.py:172-181
//   WanLayerNorm           wan/modules/model.py:89-99 (LayerNorm on bf16 input)
//   their use in a block   models/fast_dit.py:280,294,300-311
// so the fused pass equals the separate torch ops except where the order of
// the fp32 LayerNorm sums flips one bf16 rounding.  FMA contraction is off.
//
// Memory bound: one wave per token row, each lane holding dim/64 channels in
// registers between the statistics and the output; 16-byte loads and stores.
#include "launchers.h"

namespace wan {

namespace {

template <int NCH>  // 8-channel chunks per lane: dim <= 512 * NCH
__global__ __launch_bounds__(256) void adaln_kernel(const AdaLNArgs a) {
  // No contraction into FMAs: each product and sum is rounded to bf16 where the
  // separate torch ops round it (the compiler otherwise fuses ln * s1 + shift
  // across the intermediate bf16 conversion).
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= (int64_t)a.B * a.L) return;
  const int l = (int)(tok % a.L);
  const int f = l / (a.L / a.F);
  const int C = a.C, nch = C >> 3;
  const int64_t row = tok * C;
  const bf16* erow = a.e + (int64_t)f * 6 * C;
  const bf16* mrow = a.e_mod + (int64_t)f * a.mod_rows * C;

  float r[NCH][8];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const bf16x8 xv = *reinterpret_cast<const bf16x8*>(a.x + row + 8 * c);
      bf16x8 rv = xv;
      if (a.y != nullptr) {
        const bf16x8 yv = *reinterpret_cast<const bf16x8*>(a.y + row + 8 * c);
        if (a.gate_idx >= 0) {
          const bf16x8 gv = *reinterpret_cast<const bf16x8*>(erow + a.gate_idx * C + 8 * c);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const bf16 yg = (bf16)((float)yv[j] * (float)gv[j]);
            rv[j] = (bf16)((float)xv[j] + (float)yg);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) rv[j] = (bf16)((float)xv[j] + (float)yv[j]);
        }
        if (a.x_out != nullptr) *reinterpret_cast<bf16x8*>(a.x_out + row + 8 * c) = rv;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        r[i][j] = (float)rv[j];
        sum += r[i][j];
      }
    }
  }
  if (a.h_out == nullptr) return;

  const float mean = wave_sum(sum) / (float)C;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (lane + 64 * i < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = r[i][j] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)C + a.eps);

#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = rstd * (r[i][j] - mean);
      if (a.ln_w != nullptr) {
        const bf16x8 wv = *reinterpret_cast<const bf16x8*>(a.ln_w + 8 * c);
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(a.ln_b + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * (float)wv[j] + (float)bv[j];
      }
      bf16x8 hv;
      if (a.shift_idx >= 0) {
        const bf16x8 sh = *reinterpret_cast<const bf16x8*>(mrow + a.shift_idx * C + 8 * c);
        const bf16x8 sc = *reinterpret_cast<const bf16x8*>(mrow + a.scale_idx * C + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const bf16 ln = (bf16)v[j];
          const bf16 s1 = (bf16)(1.0f + (float)sc[j]);
          const bf16 t = (bf16)((float)ln * (float)s1);
          hv[j] = (bf16)((float)t + (float)sh[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[j] = (bf16)v[j];
      }
      *reinterpret_cast<bf16x8*>(a.h_out + row + 8 * c) = hv;
    }
  }
}

template <int NCH>
int launch(const AdaLNArgs& a, hipStream_t s) {
  const int64_t tokens = (int64_t)a.B * a.L;
  const int64_t grid = (tokens + 3) / 4;
  if (grid > 0x7fffffff) return set_error(2, "adaln: %lld tokens is too many", (long long)tokens);
  hipLaunchKernelGGL((adaln_kernel<NCH>), dim3((unsigned)grid), dim3(256), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "adaln launch: %s", hipGetErrorString(e));
}

}  // namespace

int launch_adaln(const AdaLNArgs& a, hipStream_t s) {
  if ((int64_t)a.B * a.L == 0) return 0;
  if (a.C <= 512) return launch<1>(a, s);
  if (a.C <= 1024) return launch<2>(a, s);
  if (a.C <= 2048) return launch<4>(a, s);
  if (a.C <= 3072) return launch<6>(a, s);
  if (a.C <= 4096) return launch<8>(a, s);
  return launch<16>(a, s);
}

}  // namespace wan
