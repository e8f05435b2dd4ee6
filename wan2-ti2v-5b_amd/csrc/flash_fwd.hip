// Flash-style attention forward for the Wan DiT on gfx950 (MI355X).
//
//   out[b, i, h, :] = sum_j softmax_j(q_i . k_j * scale) v_j   over keys j < seqlen_k[b]
//
// Semantics: F.scaled_dot_product_attention as called by _sdpa
// (models/fast_dit.py:186-189), restricted to the first `actual_seqlen_k` keys
// like wan_flash_self_attn (kernels/self_attention_nst.py:73-78,715-722), with
// the per-sample key lengths of the cross-attention call site.
//
// Design (one workgroup = NW waves = NW*32 query rows of one (batch, head)):
//  * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: the key axis is the MFMA row
//    axis, so each lane holds ONE query row (lane % 32) and 32 of the 64 keys
//    of a tile.  Row max / row sum are lane-local plus one exchange with the
//    lane 32 apart; the O rescale factor is a per-lane scalar.
//  * O^T += V^T P^T on the same MFMA: P^T comes straight out of the S^T
//    accumulator (bf16-converted, no shuffle); V^T fragments are read from the
//    natural [key][d] LDS tile with ds_read_b64_tr_b16, which returns 4 keys of
//    one channel per lane.  The key order inside a 16-key MFMA step is the
//    accumulator's row order (8*(r/4) + 4*(lane/32) + r%4); P and V use the
//    same order, and a contraction index may be permuted freely.
//  * fp32 online softmax in base 2: exp2(s * scale*log2(e) - m).
//  * K/V tiles of 64 keys are double-buffered in LDS; the next tile's global
//    loads are issued before the current tile's MFMAs and land in the other
//    buffer afterwards (one barrier per tile).
//  * Q is loaded once per wave into registers; QK-RMSNorm (given the per-token
//    inverse RMS) and the 3D-RoPE rotation are applied there, with the
//    reference's bf16 rounding points (models/fast_dit.py:145-146,169).
//  * Workgroup ids are remapped so each XCD owns contiguous query blocks of the
//    same heads (K/V reuse in that XCD's L2).
#include "common.h"

namespace wan {

namespace {

constexpr int BN = 64;                  // keys per tile
constexpr int D = kHeadDim;             // 128
constexpr int KP = D + 8;               // K tile pitch: 272 B rows, 16 rows of a b128 read hit distinct banks
constexpr int VP = D + 32;              // V tile pitch: 320 B rows, 4 rows of a tr read hit distinct banks
constexpr float kLog2e = 1.4426950408889634f;

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i16x4 lds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Query fragment for the B operand of S^T = K Q^T: lane (n32, hh) holds, for
// k-step ks, channels 16*ks + 8*hh .. +7 of query row `row`.
template <int QP>
__device__ __forceinline__ void load_q_fragment(const FlashArgs& a, int b, int h, int row,
                                                int hh, bf16x8 qf[8]) {
  if (row >= a.Lq) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = bf16x8{};
    return;
  }
  const bf16* qp = a.q.ptr + b * a.q.sb + (int64_t)row * a.q.st + h * a.q.sh;
  float inv = 1.f;
  if (QP != kQPlain) inv = a.inv_rms_q[(int64_t)b * a.Lq + row];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const int d0 = 16 * ks + 8 * hh;
    bf16x8 x = *reinterpret_cast<const bf16x8*>(qp + d0);
    if (QP != kQPlain) {
#pragma clang fp contract(off)
      const bf16x8 g = *reinterpret_cast<const bf16x8*>(a.gamma_q + h * D + d0);
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bf16 t = (bf16)((float)x[j] * inv);
        u[j] = (float)(bf16)((float)t * (float)g[j]);
      }
      if (QP == kQNormRope) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(a.cos + (int64_t)row * kRopePairs + d0 / 2);
        const f32x4 s = *reinterpret_cast<const f32x4*>(a.sin + (int64_t)row * kRopePairs + d0 / 2);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xr = u[2 * j], xi = u[2 * j + 1];
          const float p0 = xr * c[j], p1 = xi * s[j];
          const float p2 = xr * s[j], p3 = xi * c[j];
          u[2 * j] = p0 - p1;
          u[2 * j + 1] = p2 + p3;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (bf16)u[j];
    }
    qf[ks] = x;
  }
}

template <int NW, int QP>
__global__ __launch_bounds__(NW * 64, 2) void flash_fwd_kernel(const FlashArgs a) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  constexpr int CHUNKS = BN * D / 8 / NT;  // 16-byte chunks per thread per tile per tensor
  static_assert(CHUNKS * NT * 8 == BN * D, "tile must split evenly over the workgroup");

  __shared__ __attribute__((aligned(16))) bf16 k_lds[2][BN * KP];
  __shared__ __attribute__((aligned(16))) bf16 v_lds[2][BN * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n32 = lane & 31, hh = lane >> 5;

  const int num_m = (a.Lq + BM - 1) / BM;
  const int pid = xcd_remap(blockIdx.x, gridDim.x);
  const int mblk = pid % num_m;
  const int bh = pid / num_m;
  const int b = bh / a.H, h = bh - b * a.H;

  int len = a.seqlen_all;
  if (a.seqlen_k != nullptr) len = min(max(a.seqlen_k[b], 0), a.Lk);
  const int ntiles = (len + BN - 1) / BN;

  const int qrow = mblk * BM + wave * 32 + n32;
  bf16x8 qf[8];
  load_q_fragment<QP>(a, b, h, qrow, hh, qf);

  const bf16* kbase = a.k.ptr + b * a.k.sb + h * a.k.sh;
  const bf16* vbase = a.v.ptr + b * a.v.sb + h * a.v.sh;

  uint4 kr[CHUNKS], vr[CHUNKS];
  auto gload = [&](int t) {
#pragma unroll
    for (int j = 0; j < CHUNKS; ++j) {
      const int c = tid + NT * j;
      const int row = c >> 4, col = (c & 15) * 8;
      const int key = t * BN + row;
      if (key < len) {
        kr[j] = *reinterpret_cast<const uint4*>(kbase + (int64_t)key * a.k.st + col);
        vr[j] = *reinterpret_cast<const uint4*>(vbase + (int64_t)key * a.v.st + col);
      } else {
        kr[j] = uint4{0, 0, 0, 0};
        vr[j] = uint4{0, 0, 0, 0};
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < CHUNKS; ++j) {
      const int c = tid + NT * j;
      const int row = c >> 4, col = (c & 15) * 8;
      *reinterpret_cast<uint4*>(&k_lds[buf][row * KP + col]) = kr[j];
      *reinterpret_cast<uint4*>(&v_lds[buf][row * VP + col]) = vr[j];
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md) o[md] = f32x16{};
  float m_run = -INFINITY;  // running max, in scale*log2(e) units
  float l_run = 0.f;        // this lane's partial row sum (its 32 keys of each tile)
  const float sl2 = a.scale * kLog2e;

  // Source lane of a transposed V read: key row (lane%16)/4 of a 4-key group,
  // channels 4*(lane%4) .. +3 of a 16-channel group.
  const int tr_key = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const bf16* Kt = k_lds[buf];
    const bf16* Vt = v_lds[buf];

    // S^T[key][query] for keys 0..31 (s0) and 32..63 (s1) of this tile.
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(Kt + n32 * KP + 16 * ks + 8 * hh);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(Kt + (32 + n32) * KP + 16 * ks + 8 * hh);
      s0 = mfma32(a0, qf[ks], s0);
      s1 = mfma32(a1, qf[ks], s1);
    }

    const int kt = t * BN;
    if (kt + BN > len) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (key >= len) s0[r] = -INFINITY;
        if (key + 32 >= len) s1[r] = -INFINITY;
      }
    }

    float mx = s0[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s0[r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * sl2);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;

    bf16x8 pb[4];
    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s0[r], sl2, -m_new));
      rs += p;
      pb[r >> 3][r & 7] = (bf16)p;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s1[r], sl2, -m_new));
      rs += p;
      pb[2 + (r >> 3)][r & 7] = (bf16)p;
    }
    l_run = l_run * alpha + rs;
#pragma unroll
    for (int md = 0; md < 4; ++md) o[md] *= alpha;

    // O^T[d][query] += V^T[d][key] P^T[key][query], 16 keys per step.
#pragma unroll
    for (int ksp = 0; ksp < 4; ++ksp) {
#pragma unroll
      for (int md = 0; md < 4; ++md) {
        const bf16* vp = Vt + (16 * ksp + tr_key) * VP + 32 * md + tr_col;
        const i16x4 lo = lds_read_tr(vp);
        const i16x4 hi = lds_read_tr(vp + 8 * VP);
        const bf16x8 av = __builtin_bit_cast(
            bf16x8, (short __attribute__((ext_vector_type(8)))){lo[0], lo[1], lo[2], lo[3],
                                                                hi[0], hi[1], hi[2], hi[3]});
        o[md] = mfma32(av, pb[ksp], o[md]);
      }
    }

    if (t + 1 < ntiles) lstore(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qrow < a.Lq) {
    bf16* op = a.o + b * a.o_sb + (int64_t)qrow * a.o_st + h * a.o_sh;
#pragma unroll
    for (int md = 0; md < 4; ++md) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (bf16)(o[md][4 * g + e] * inv_l);
        *reinterpret_cast<bf16x4*>(op + 32 * md + 8 * g + 4 * hh) = w;
      }
    }
  }
}

template <int NW, int QP>
int launch_nw_qp(const FlashArgs& a, hipStream_t s) {
  constexpr int BM = NW * 32;
  const int64_t num_m = (a.Lq + BM - 1) / BM;
  const int64_t grid = num_m * a.B * a.H;
  if (grid > 0x7fffffff) return set_error(2, "flash_fwd: grid of %lld workgroups too large", (long long)grid);
  hipLaunchKernelGGL((flash_fwd_kernel<NW, QP>), dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "flash_fwd launch: %s", hipGetErrorString(e));
}

}  // namespace

int launch_flash_fwd(const FlashArgs& a, hipStream_t s) {
  if (a.B == 0 || a.H == 0 || a.Lq == 0) return 0;
  switch (a.qprep) {
    case kQPlain: return launch_nw_qp<4, kQPlain>(a, s);
    case kQNorm: return launch_nw_qp<4, kQNorm>(a, s);
    case kQNormRope: return launch_nw_qp<4, kQNormRope>(a, s);
    default: return set_error(1, "flash_fwd: unknown q preparation %d", a.qprep);
  }
}

}  // namespace wan
