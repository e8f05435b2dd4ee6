// Flash-style attention forward for the Wan DiT on gfx950 (MI355X).
//
//   out[b, i, h, :] = sum_j softmax_j(q_i . k_j * scale) v_j   over keys j < seqlen_k[b]
//
// Semantics: F.scaled_dot_product_attention as called by _sdpa
// (models/fast_dit.py:186-189), restricted to the first `actual_seqlen_k` keys
// like wan_flash_self_attn (kernels/self_attention_nst.py:73-78,715-722), with
// the per-sample key lengths of the cross-attention call site.
//
// Design (one workgroup = 8 waves = 256 query rows of one (batch, head); one
// workgroup per CU at up to 256 VGPRs per wave):
//  * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: the key axis is the MFMA row
//    axis, so each lane holds ONE query row (lane % 32) and 32 of the 64 keys
//    of a tile.  Row max / row sum are lane-local plus one exchange with the
//    lane 32 apart (v_permlane32_swap); the O rescale factor is a per-lane scalar.
//  * O^T += V^T P^T on the same MFMA: P^T comes straight out of the S^T
//    accumulator (bf16-converted, no shuffle); V^T fragments are read from the
//    natural [key][d] LDS tile with ds_read_b64_tr_b16, which returns 4 keys of
//    one channel per lane.  The key order inside a 16-key MFMA step is the
//    accumulator's row order (8*(r/4) + 4*(lane/32) + r%4); P and V use the
//    same order, and a contraction index may be permuted freely.
//  * fp32 online softmax in base 2: p = exp2(s * scale*log2(e) - m).  The
//    reference point m is not the exact running max: a tile is exponentiated
//    against the current m, and only when some lane's sum of the tile's p
//    exceeds kSumBound (or is inf / NaN) is the tile's exact max taken, m
//    moved and O, l rescaled (the first tile always; later tiles rarely).
//    Otherwise every p <= kSumBound and the stale reference point cancels in
//    O / l exactly.  l sums the bf16-rounded p that the PV MFMAs consume.
//  * K/V tiles of 64 keys go global -> LDS directly (global_load_lds_dwordx4),
//    double-buffered, 16-byte chunks XOR-swizzled per row so the MFMA operand
//    reads are bank-conflict free without padding.  Software pipeline: while
//    the softmax of tile j runs on the VALU, the S^T MFMAs of tile j+1 and the
//    loads of tiles j+1 (V) and j+2 (K) are in flight.  One barrier per tile;
//    with 8 waves a ring of four K and four V tiles (128 KB) lets the barrier
//    come every second tile, the loads of a tile pair going out one pair ahead.
//    In program order the S^T MFMAs of tile j+1 alternate with the exp2 /
//    convert / sum of tile j (two MFMAs and four exponentials per k-step), and
//    K and V^T operand fragments are read one MFMA ahead.  The tile copies are
//    issued from inline asm, out of sight of the compiler's wait counting, so
//    the LDS operand reads wait only for themselves.
//  * Q is loaded once per wave into registers; QK-RMSNorm (given the per-token
//    inverse RMS) and the 3D-RoPE rotation are applied there, with the
//    reference's bf16 rounding points (models/fast_dit.py:145-146,169).  The
//    wave's 32 cos and sin rows come through LDS (1 KB copies, before the K/V
//    tiles occupy it): read per lane from global memory they cost each wave
//    512 scattered 32-byte requests.  Without RoPE, the 4-wave kernel stages
//    the q rows the same way.
//  * The output tile goes back through LDS as well and leaves as whole 128-byte
//    row segments, with non-temporal stores.
//  * Workgroup ids are remapped so each XCD owns contiguous query blocks of the
//    same heads (K/V reuse in that XCD's L2); with per-sample key lengths the
//    batch index varies fastest instead, balancing long and short samples
//    over the XCDs.
#include "common.h"


namespace wan {

namespace {

constexpr int BN = 64;                  // keys per tile
constexpr int kWaves = 8;               // waves per workgroup: 256 query rows, one workgroup per CU
constexpr int D = kHeadDim;             // 128
constexpr int kTileElems = BN * D;      // one K or V tile: 64 rows of 256 B
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSumBound = 65536.0f;   // per-lane tile sum of P that forces a rescale
constexpr int kShortTableBytes = 16384; // persistent short-key kernel: gammas + key lengths

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i16x4 lds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of a lane's value and the value of the lane 32 apart (same query row)
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS tile layouts (element offsets).  Row r = key, 16 chunks of 8 channels.
//  K: chunk c of row r sits at position c ^ (r & 15): the 16 rows read by a
//     b128 phase land on 16 distinct bank groups.
//  V: chunk c of row r sits at position c ^ 4*(r & 3): the 4 rows x 4 chunks
//     of a transposed-read phase land on 16 distinct bank groups.
__device__ __forceinline__ int k_swz(int row) { return row & 15; }
__device__ __forceinline__ int v_swz(int row) { return (row & 3) << 2; }

// Query fragment for the B operand of S^T = K Q^T: lane (n32, hh) holds, for
// k-step ks, channels 16*ks + 8*hh .. +7 of query row `row`.
template <int QP>
__device__ __forceinline__ void load_q_fragment(const FlashArgs& a, int b, int h, int row,
                                                int hh, bf16x8 qf[8], const char* cos_lds,
                                                const char* sin_lds, int n32,
                                                const char* q_lds = nullptr) {
  if (row >= a.Lq) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = bf16x8{};
    return;
  }
  const bf16* qp = a.q.ptr + b * a.q.sb + (int64_t)row * a.q.st + h * a.q.sh;
  float inv = 1.f;
  if (QP != kQPlain) inv = a.inv_rms_q[(int64_t)b * a.Lq + row];
  bf16x8 x[8], g[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const int d0 = 16 * ks + 8 * hh;
    if (q_lds == nullptr) x[ks] = *reinterpret_cast<const bf16x8*>(qp + d0);
    if (QP != kQPlain) g[ks] = *reinterpret_cast<const bf16x8*>(a.gamma_q + h * D + d0);
  }
  // the staged rows (copies issued by this wave before) have landed
  if (QP == kQNormRope || q_lds != nullptr) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (q_lds != nullptr) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      x[ks] = *reinterpret_cast<const bf16x8*>(q_lds + n32 * 256 + (((2 * ks + hh) ^ (n32 & 15)) << 4));
  }
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (QP != kQPlain) {
#pragma clang fp contract(off)
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bf16 t = (bf16)((float)x[ks][j] * inv);
        u[j] = (float)(bf16)((float)t * (float)g[ks][j]);
      }
      if (QP == kQNormRope) {
        // chunk (2 ks + hh) of row n32 sits at position chunk ^ (n32 & 15)
        const int off = n32 * 256 + (((2 * ks + hh) ^ (n32 & 15)) << 4);
        const f32x4 c = *reinterpret_cast<const f32x4*>(cos_lds + off);
        const f32x4 s = *reinterpret_cast<const f32x4*>(sin_lds + off);
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
      for (int j = 0; j < 8; ++j) x[ks][j] = (bf16)u[j];
    }
    qf[ks] = x[ks];
  }
}

// 16-byte global -> LDS copies (global_load_lds_dwordx4): lane l writes LDS
// bytes m0 + 16 l .. +15.  Issued from inline asm so that the compiler's
// wait-count bookkeeping does not see them: it would otherwise treat every LDS
// read that follows an in-flight copy as out of order and wait for all of
// them (lgkmcnt(0)) before each use.  Completion is the kernel's own business:
// every tile is waited for (s_waitcnt vmcnt(0)) before the barrier that
// publishes it.  The LDS address is an operand bound to m0 ("{m0}"), so the
// compiler writes m0 itself and knows its value; the s_nop covers the wait
// state between an m0 write and an LDS-DMA that reads it.
__device__ __forceinline__ uint32_t lds_addr(const bf16* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) bf16*)p;
}
__device__ __forceinline__ void dma16_saddr(const char* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_vaddr(const char* vaddr, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(vaddr), "{m0}"(lds) : "memory");
}

// Copies rows [row0, row0 + 32) of a table with 256-byte rows into 8 KB of
// LDS, 1 KB (four rows) per copy: chunk c of row r lands at position
// c ^ (r & 15), so the per-lane 16-byte reads of one chunk across 16 rows
// are conflict free.  Rows past last_row repeat last_row.
__device__ __forceinline__ void stage_rows32(const char* base, int64_t row_bytes, int row0, int last_row,
                                             bf16* lds, int lane) {
  const uint32_t l0 = lds_addr(lds);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = 4 * i + (lane >> 4);
    const int row = min(row0 + rr, last_row);
    const int c = (lane & 15) ^ (rr & 15);
    dma16_vaddr(base + (int64_t)row * row_bytes + c * 16, l0 + i * 1024);
  }
}

template <int NW>
struct TileLoader {
  // Wave `wave` issues the 1 KB blocks i = wave, wave + NW, ... of a 16 KB
  // tile; lane l fills LDS row 4i + l/16, position l%16, with the chunk that
  // the row's swizzle puts there.  Full tiles are addressed as a wave-uniform
  // base plus a 32-bit per-lane byte offset (the scalar-base form of the
  // load: no 64-bit per-lane address is kept live).
  static constexpr int kPerWave = 16 / NW;
  const char* base;              // (batch, head) origin of the K or V tensor
  int64_t stride;                // token stride (elements)
  uint32_t lane_off[kPerWave];   // bytes: row * stride + source column, for a full tile
  bool is_k;

  __device__ __forceinline__ int row_of(int wave, int lane, int u) const {
    return 4 * (wave + NW * u) + (lane >> 4);
  }
  __device__ __forceinline__ int col_of(int row, int lane) const {
    return ((lane & 15) ^ (is_k ? k_swz(row) : v_swz(row))) * 8;
  }

  __device__ void init(const bf16* b, int64_t st, int wave, int lane, bool k) {
    base = reinterpret_cast<const char*>(b);
    stride = st;
    is_k = k;
#pragma unroll
    for (int u = 0; u < kPerWave; ++u) {
      const int row = row_of(wave, lane, u);
      lane_off[u] = (uint32_t)(row * st + col_of(row, lane)) * 2u;
    }
  }

  // Issue the loads of tile t (keys t*BN ..) into `dst`.  In the last tile,
  // rows past len-1 repeat key len-1 (finite data whose scores are masked).
  __device__ __forceinline__ void issue(int t, int len, bf16* dst, int wave, int lane) const {
    const int k0 = t * BN;
    if (k0 + BN <= len) {
      const char* tb = base + (int64_t)k0 * stride * 2;
#pragma unroll
      for (int u = 0; u < kPerWave; ++u) {
        // keep the 32 -> 64-bit extension next to the load (not hoisted out of
        // the tile loop) so instruction selection sees sgpr + zext(vgpr)
        dma16_saddr(tb, lane_off[u], lds_addr(dst + (wave + NW * u) * 512));
      }
    } else {
#pragma unroll
      for (int u = 0; u < kPerWave; ++u) {
        const int row = row_of(wave, lane, u);
        const int key = min(k0 + row, len - 1);
        dma16_vaddr(base + ((int64_t)key * stride + col_of(row, lane)) * 2,
                    lds_addr(dst + (wave + NW * u) * 512));
      }
    }
  }
};

// Per-wave state and tile arithmetic of the attention loop: the O^T accumulator,
// the running reference max m_run (scale*log2(e) units) and this lane's partial row
// sum l_run (its 32 keys of each tile), the Q fragments, and the lane-constant LDS
// operand offsets.  Everything is force-inlined into the kernels that use it.
struct TileCore {
  f32x16 o[4];
  float m_run;
  float l_run;
  float sl2;       // softmax scale * log2(e)
  bf16x8 qf[8];    // B operand of S^T = K Q^T: query row lane % 32, channels 16 ks + 8 hh ..
  int k_rd[8];
  int v_rd[4];
  int hh;

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int md = 0; md < 4; ++md) o[md] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;
  }

  __device__ __forceinline__ void set_offsets(int lane, float scale) {
    const int n32 = lane & 31;
    hh = lane >> 5;
    sl2 = scale * kLog2e;
    // rows n32 and 32 + n32 share the swizzle (row & 15): one offset per k-step
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) k_rd[ks] = n32 * D + (((2 * ks + hh) ^ k_swz(n32)) << 3);
    const int tr_row = 4 * hh + ((lane & 15) >> 2);  // + 16*ksp + 8*r
    const int tr_chunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);  // + 4*md
    const int tr_sub = 4 * (lane & 1);
    const int tr_x = v_swz(tr_row);  // (row & 3) is the same for every ksp, r
#pragma unroll
    for (int md = 0; md < 4; ++md) v_rd[md] = tr_row * D + (((4 * md + tr_chunk) ^ tr_x) << 3) + tr_sub;
  }

  // S^T of one 64-key tile: s0 holds keys 0..31, s1 keys 32..63 (accumulator row order)
  __device__ __forceinline__ void qk(const bf16* Kt, f32x16& s0, f32x16& s1) const {
    s0 = f32x16{};
    s1 = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[ks]);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[ks] + 32 * D);
      s0 = mfma32(a0, qf[ks], s0);
      s1 = mfma32(a1, qf[ks], s1);
    }
  }

  // P = exp2(S * scale*log2e - m_run) in bf16, and this lane's sum of P
  // (of the bf16 values the PV MFMAs use; v_dot2 against (1, 1)).
  // Used off the hot loop only (the last tile and the rescale path): each
  // quarter of the tile is a scheduling region of its own, which bounds the
  // exponentials in flight (and the register pressure) at eight.
  __device__ __forceinline__ float exp_tile(const f32x16& s0, const f32x16& s1, bf16x8 pb[4]) const {
    const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x16& sv = i < 2 ? s0 : s1;
#pragma unroll
      for (int j = 0; j < 8; ++j) pb[i][j] = (bf16)fast_exp2(fmaf(sv[8 * (i & 1) + j], sl2, -m_run));
      acc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb[i], pb[i], 0, 1), one, acc[i], false);
      acc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb[i], pb[i], 2, 3), one, acc[i], false);
      acc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb[i], pb[i], 4, 5), one, acc[i], false);
      acc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb[i], pb[i], 6, 7), one, acc[i], false);
      __builtin_amdgcn_sched_barrier(0);
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }

  // Completes the softmax numerator of a tile whose P was computed against
  // the current reference max with lane sum rs.  Only if some lane's sum
  // exceeds kSumBound (or is inf / NaN: the first tile, where m_run is -inf)
  // does the wave take the tile's exact row max, rescale O and l, and
  // exponentiate again; afterwards every p <= 1.
  __device__ __forceinline__ void finish(const f32x16& s0, const f32x16& s1, float rs, bf16x8 pb[4]) {
    if (__builtin_amdgcn_ballot_w64(!(rs <= kSumBound)) != 0) {
      float mx = fmaxf(s0[0], s0[1]);
#pragma unroll
      for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s0[r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
      const float m_new = fmaxf(m_run, pair_max(mx) * sl2);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int md = 0; md < 4; ++md) o[md] *= alpha;
      rs = exp_tile(s0, s1, pb);
    }
    l_run += rs;
  }

  // The reference point from the exact row max of the first tile's scores.  Left at -inf,
  // the first tile's exponentials overflow in qk_exp and finish() computes them again
  // (for an item of two tiles, half of all its exponentials).  Keys past the length in
  // a partial first tile are copies of the last valid key, so they do not raise the max.
  __device__ __forceinline__ void init_max(const f32x16& s0, const f32x16& s1) {
    float mx = fmaxf(s0[0], s0[1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s0[r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
    m_run = pair_max(mx) * sl2;
  }

  // Sets the scores of keys >= len to -inf (a partial last tile starting at key kt).
  __device__ __forceinline__ void mask_tile(f32x16& s0, f32x16& s1, int kt, int len) const {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kt + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key >= len) s0[r] = -INFINITY;
      if (key + 32 >= len) s1[r] = -INFINITY;
    }
  }

  // The MFMAs of S(next) = K Q^T, interleaved in program order with the
  // exponentials of the current tile's S (c0, c1): per k-step two MFMAs and
  // elements 2ks, 2ks+1 of each half (4 fma + 4 exp2 + 2 cvt + 2 dot2).  K
  // fragments are read one k-step ahead.  Returns this lane's sum of P.
  __device__ __forceinline__ float qk_exp(const bf16* Kt, f32x16& n0, f32x16& n1, const f32x16& c0,
                                          const f32x16& c1, bf16x8 pb[4]) const {
    const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
    float acc0 = 0.f, acc1 = 0.f;
    bf16x8 a0 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[0]);
    bf16x8 a1 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[0] + 32 * D);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      bf16x8 b0, b1;
      if (ks < 7) {
        b0 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[ks + 1]);
        b1 = *reinterpret_cast<const bf16x8*>(Kt + k_rd[ks + 1] + 32 * D);
      }
      n0 = mfma32(a0, qf[ks], ks == 0 ? f32x16{} : n0);
      n1 = mfma32(a1, qf[ks], ks == 0 ? f32x16{} : n1);
      const int r = 2 * ks;
      const bf16x2 u = {(bf16)fast_exp2(fmaf(c0[r], sl2, -m_run)),
                        (bf16)fast_exp2(fmaf(c0[r + 1], sl2, -m_run))};
      const bf16x2 w = {(bf16)fast_exp2(fmaf(c1[r], sl2, -m_run)),
                        (bf16)fast_exp2(fmaf(c1[r + 1], sl2, -m_run))};
      pb[ks >> 2][2 * (ks & 3)] = u[0];
      pb[ks >> 2][2 * (ks & 3) + 1] = u[1];
      pb[2 + (ks >> 2)][2 * (ks & 3)] = w[0];
      pb[2 + (ks >> 2)][2 * (ks & 3) + 1] = w[1];
      acc0 = __builtin_amdgcn_fdot2_f32_bf16(u, one, acc0, false);
      acc1 = __builtin_amdgcn_fdot2_f32_bf16(w, one, acc1, false);
      if (ks < 7) {
        a0 = b0;
        a1 = b1;
      }
    }
    return acc0 + acc1;
  }

  // O^T += V^T P^T, V^T fragments read one MFMA ahead
  __device__ __forceinline__ void pv(const bf16x8 pb[4], const bf16* Vt) {
    auto vfrag = [&](int i) -> bf16x8 {
      const bf16* vp = Vt + 16 * (i >> 2) * D + v_rd[i & 3];
      const i16x4 lo = lds_read_tr(vp);
      const i16x4 hi = lds_read_tr(vp + 8 * D);
      return __builtin_bit_cast(bf16x8, (short __attribute__((ext_vector_type(8)))){
                                            lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
    };
    bf16x8 cur = vfrag(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      bf16x8 nxt;
      if (i < 15) nxt = vfrag(i + 1);
      o[i & 3] = mfma32(cur, pb[i >> 2], o[i & 3]);
      if (i < 15) cur = nxt;
    }
  }

  // This wave's output tile (32 rows x 128 channels, divided by the row sum),
  // staged through 4 KB of LDS at `stage` so that each store instruction writes
  // whole 128-byte row segments (8 rows x 128 B) instead of 8-byte pieces of 32
  // rows.  Two 64-channel halves; rows hold 8 chunks of 16 B, chunk c of row r at
  // position c ^ (r & 7).  Non-temporal stores: the output is written once and not
  // re-read here, so it should not displace K/V lines other workgroups still read.
  __device__ __forceinline__ void store_out(bf16* stage, bf16* obase, int64_t o_st, int row0, int Lq,
                                            int lane) const {
    const int n32 = lane & 31, half_lane = lane >> 5;   // (set_offsets may not have run)
    const float l_tot = pair_sum(l_run);
    const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = (bf16)(o[2 * half + mm][4 * g + e] * inv_l);
          const int c = 4 * mm + g;  // lane holds channels 8c + 4hh .. +3 of row n32
          *reinterpret_cast<bf16x4*>(stage + n32 * 64 + ((c ^ (n32 & 7)) << 3) + 4 * half_lane) = w;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 8 * j + (lane >> 3), c = lane & 7;
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(stage + r * 64 + ((c ^ (r & 7)) << 3));
        if (row0 + r < Lq)
          __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(obase + (int64_t)(row0 + r) * o_st + 64 * half + 8 * c));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
};

template <int NW, int QP>
__global__ __launch_bounds__(NW * 64, 2) void flash_fwd_kernel(const FlashArgs a) {
  constexpr int BM = NW * 32;

  // K and V tiles resident per workgroup: a ring of four each (128 KB) with
  // 8 waves, which run one workgroup per CU; two each (64 KB) with 4 waves, so
  // that two workgroups fit a CU.  After the last tile the first two K
  // buffers stage the output.
  constexpr int RING = NW == 8 ? 4 : 2;
  __shared__ __attribute__((aligned(1024))) bf16 k_lds[RING][kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds[RING][kTileElems];
  // with the ring of four, 32 KB more: room for the RoPE row staging while
  // the first K and V tiles are already being copied
  __shared__ __attribute__((aligned(1024))) bf16 x_lds[RING == 4 ? 2 * kTileElems : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n32 = lane & 31, hh = lane >> 5;

  const int num_m = (a.Lq + BM - 1) / BM;
  const int pid = xcd_remap(blockIdx.x, gridDim.x);
  int mblk, b, h;
  if (a.seqlen_k == nullptr) {
    // (b, h) major: the query blocks of one head run together on one XCD and
    // share its K/V through that XCD's L2
    mblk = pid % num_m;
    const int bh = pid / num_m;
    b = bh / a.H;
    h = bh - b * a.H;
  } else {
    // per-sample key lengths: batch fastest, so every XCD receives the same
    // mix of long and short samples (the K/V of these calls are small)
    b = pid % a.B;
    const int rest = pid / a.B;
    mblk = rest % num_m;
    h = rest / num_m;
  }

  int len = a.seqlen_all;
  if (a.seqlen_k != nullptr) len = min(max(a.seqlen_k[b], 0), a.Lk);
  const int ntiles = (len + BN - 1) / BN;

  const int qrow = mblk * BM + wave * 32 + n32;
  TileCore c;
  c.reset();

  if (ntiles > 0) {
    TileLoader<NW> kl, vl;
    kl.init(a.k.ptr + b * a.k.sb + h * a.k.sh, a.k.st, wave, lane, true);
    vl.init(a.v.ptr + b * a.v.sb + h * a.v.sh, a.v.st, wave, lane, false);
    // RoPE tables: this wave's 32 cos and sin rows go through LDS and are read
    // back per lane.  With the ring of four they use buffers 1-3 and the extra
    // 32 KB while K0 and V0 are already being copied; with two buffers they use
    // all of them and the tiles follow.
    if constexpr (QP == kQNormRope) {
      const int row0w = mblk * BM + wave * 32;
      bf16 *cos_st, *sin_st;
      if constexpr (RING == 4) {
        kl.issue(0, len, k_lds[0], wave, lane);
        vl.issue(0, len, v_lds[0], wave, lane);
        cos_st = wave < 6 ? &k_lds[1 + wave / 2][0] + (wave & 1) * 4096 : &x_lds[0] + (wave - 6) * 4096;
        sin_st = wave < 6 ? &v_lds[1 + wave / 2][0] + (wave & 1) * 4096 : &x_lds[8192] + (wave - 6) * 4096;
      } else {
        cos_st = &k_lds[0][0] + wave * 4096;
        sin_st = &v_lds[0][0] + wave * 4096;
      }
      stage_rows32(reinterpret_cast<const char*>(a.cos), kRopePairs * 4, row0w, a.Lq - 1, cos_st, lane);
      stage_rows32(reinterpret_cast<const char*>(a.sin), kRopePairs * 4, row0w, a.Lq - 1, sin_st, lane);
      load_q_fragment<QP>(a, b, h, qrow, hh, c.qf, reinterpret_cast<const char*>(cos_st),
                          reinterpret_cast<const char*>(sin_st), n32);
      // every wave's staging copies have landed (also those of a wave whose rows
      // are all past Lq) and every wave is done reading them before tiles are
      // copied over them
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if constexpr (RING == 4) {
        if (ntiles > 1) {
          kl.issue(1, len, k_lds[1], wave, lane);
          vl.issue(1, len, v_lds[1], wave, lane);
        }
        if (ntiles > 2) kl.issue(2, len, k_lds[2], wave, lane);
      } else {
        kl.issue(0, len, k_lds[0], wave, lane);
        vl.issue(0, len, v_lds[0], wave, lane);
        if (ntiles > 1) kl.issue(1, len, k_lds[1], wave, lane);
      }
    } else if constexpr (RING == 2) {
      // K0 and K1 go out first; the wave's 32 q rows come through the V
      // buffers (1 KB copies instead of 32-row scattered loads), then V0
      kl.issue(0, len, k_lds[0], wave, lane);
      if (ntiles > 1) kl.issue(1, len, k_lds[1], wave, lane);
      const int row0w = mblk * BM + wave * 32;
      bf16* q_st = &v_lds[0][0] + wave * 4096;
      stage_rows32(reinterpret_cast<const char*>(a.q.ptr + b * a.q.sb + h * a.q.sh), a.q.st * 2, row0w,
                   a.Lq - 1, q_st, lane);
      load_q_fragment<QP>(a, b, h, qrow, hh, c.qf, nullptr, nullptr, n32, reinterpret_cast<const char*>(q_st));
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // every wave is done with its staged rows before V0 lands there
      vl.issue(0, len, v_lds[0], wave, lane);
    } else {
      // the first tiles go out before the Q rows are read: the two latencies overlap
      kl.issue(0, len, k_lds[0], wave, lane);
      vl.issue(0, len, v_lds[0], wave, lane);
      if (ntiles > 1) kl.issue(1, len, k_lds[1], wave, lane);
      if (ntiles > 1) vl.issue(1, len, v_lds[1], wave, lane);
      if (ntiles > 2) kl.issue(2, len, k_lds[2], wave, lane);
      load_q_fragment<QP>(a, b, h, qrow, hh, c.qf, nullptr, nullptr, n32);
    }

    c.set_offsets(lane, a.scale);

    // One pipelined step on tile t (not the last tile): the loads of K(t+2)
    // and V(t+1); the MFMAs of S(t+1) = K(t+1) Q^T, the softmax of S(t) and
    // O += V(t) P(t).  Tile t lives in buffers t%2; the buffer arguments are
    // static per call.
    auto step = [&](int t, bf16* k_fill, bf16* v_fill, const bf16* k_next, const bf16* v_cur,
                    f32x16& c0, f32x16& c1, f32x16& n0, f32x16& n1) {
      bf16x8 pb[4];
      c.finish(c0, c1, c.qk_exp(k_next, n0, n1, c0, c1, pb), pb);
      // the copies go out between the softmax and PV, as in the other loops
      if (t + 2 < ntiles) kl.issue(t + 2, len, k_fill, wave, lane);
      vl.issue(t + 1, len, v_fill, wave, lane);
      c.pv(pb, v_cur);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };

    f32x16 sa0, sa1, sb0, sb1;
    if constexpr ((QP == kQNormRope && RING == 4) || (QP != kQNormRope && RING == 2)) {
      // the staging barrier published the first K tile(s) (and V0 with the
      // ring of four); the tiles issued after it land while S(0) is computed,
      // and this barrier publishes them and frees K0
      c.qk(k_lds[0], sa0, sa1);
      c.init_max(sa0, sa1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    } else {
      // prologue: S(0) once the first tiles have landed
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      c.qk(k_lds[0], sa0, sa1);
      c.init_max(sa0, sa1);
      __syncthreads();  // every wave is done with K0 before it is overwritten
    }

    int t = 0;
    const bf16* v_last = v_lds[0];
    if constexpr (RING == 2) {
      for (; t + 2 < ntiles; t += 2) {
        step(t, k_lds[0], v_lds[1], k_lds[1], v_lds[0], sa0, sa1, sb0, sb1);
        step(t + 1, k_lds[1], v_lds[0], k_lds[0], v_lds[1], sb0, sb1, sa0, sa1);
      }
      // One full tile may remain before the last; then the last tile's scores are
      // moved into sa so that a single copy of the last-tile code follows (its
      // V buffer is picked at run time; every load has landed by then).
      if (t + 1 < ntiles) {
        step(t, k_lds[0], v_lds[1], k_lds[1], v_lds[0], sa0, sa1, sb0, sb1);
        sa0 = sb0;
        sa1 = sb1;
        v_last = v_lds[1];
        ++t;
      }
    } else {
      // Ring of four: a barrier after every second step only.  An even step t
      // issues the next pair's tiles, K(t+3), K(t+4), V(t+2), V(t+3), into the
      // buffers that the previous pair finished reading; the odd step after it
      // waits for them and publishes them with the barrier.
      auto step4 = [&](int t, int odd, const bf16* k_next, const bf16* v_cur, bf16* kf3, bf16* kf4,
                       bf16* vf2, bf16* vf3, f32x16& c0, f32x16& c1, f32x16& n0, f32x16& n1) {
        bf16x8 pb[4];
        c.finish(c0, c1, c.qk_exp(k_next, n0, n1, c0, c1, pb), pb);
        // the copies go out between the softmax and PV: issued at the step's start, their
        // burst held up both waves of each SIMD at once (2.3-2.7% slower at L=7854)
        if (!odd) {
          if (t + 3 < ntiles) kl.issue(t + 3, len, kf3, wave, lane);
          if (t + 4 < ntiles) kl.issue(t + 4, len, kf4, wave, lane);
          if (t + 2 < ntiles) vl.issue(t + 2, len, vf2, wave, lane);
          if (t + 3 < ntiles) vl.issue(t + 3, len, vf3, wave, lane);
        }
        c.pv(pb, v_cur);
        if (odd) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
        }
      };
      for (; t + 4 < ntiles; t += 4) {
        step4(t, 0, k_lds[1], v_lds[0], k_lds[3], k_lds[0], v_lds[2], v_lds[3], sa0, sa1, sb0, sb1);
        step4(t + 1, 1, k_lds[2], v_lds[1], nullptr, nullptr, nullptr, nullptr, sb0, sb1, sa0, sa1);
        step4(t + 2, 0, k_lds[3], v_lds[2], k_lds[1], k_lds[2], v_lds[0], v_lds[1], sa0, sa1, sb0, sb1);
        step4(t + 3, 1, k_lds[0], v_lds[3], nullptr, nullptr, nullptr, nullptr, sb0, sb1, sa0, sa1);
      }
      // the remaining full tiles (at most three), buffers picked at run time
      for (; t + 1 < ntiles; ++t) {
        const int j = t & 3;
        step4(t, t & 1, k_lds[(j + 1) & 3], v_lds[j], k_lds[(j + 3) & 3], k_lds[j], v_lds[(j + 2) & 3],
              v_lds[(j + 3) & 3], sa0, sa1, sb0, sb1);
        sa0 = sb0;
        sa1 = sb1;
      }
      v_last = v_lds[t & 3];
    }
    // the last tile, its keys >= len masked when it is partial
    if (ntiles * BN > len) c.mask_tile(sa0, sa1, t * BN, len);
    bf16x8 pb[4];
    c.finish(sa0, sa1, c.exp_tile(sa0, sa1, pb), pb);
    c.pv(pb, v_last);
    // the output staging below overwrites K buffers that a slower wave may
    // still read in its last step when that step ended without a barrier
    if constexpr (RING == 4) __syncthreads();
  }

  // Output store, staged through the K buffers: they are free here (their last
  // reads came before the last barrier, and no load into them is in flight).
  bf16* stage = (wave < 4 ? k_lds[0] : k_lds[1]) + (wave & 3) * 2048;
  c.store_out(stage, a.o + b * a.o_sb + h * a.o_sh, a.o_st, mblk * BM + wave * 32, a.Lq, lane);
}

// Explicit instantiations: without them clang emits the host launch stubs of
// only some of these (lambda-using) kernel template instances.
template __global__ void flash_fwd_kernel<kWaves, kQPlain>(const FlashArgs);
template __global__ void flash_fwd_kernel<kWaves, kQNorm>(const FlashArgs);
template __global__ void flash_fwd_kernel<kWaves, kQNormRope>(const FlashArgs);
template __global__ void flash_fwd_kernel<4, kQPlain>(const FlashArgs);
template __global__ void flash_fwd_kernel<4, kQNorm>(const FlashArgs);
template __global__ void flash_fwd_kernel<4, kQNormRope>(const FlashArgs);

// ---------------------------------------------------------------------------
// Short keys (<= kShortKeys, the cross-attention's text keys) with per-sample key
// lengths and no RoPE on the query: a persistent kernel.  A workgroup has 4 waves
// (128 query rows of one (batch, head) per item) and two run per CU.  Items of a
// short sample are mostly start-up (query rows, first K/V tiles) and output store;
// here, once an item's last S MFMAs are done, the next item's first two K tiles are
// copied into the (then free) K buffers and its query rows loaded into the (then
// free) Q registers, so that start-up overlaps the item's last tile; they are waited
// for before the item's output stores, and nothing after the stores loads from global
// memory before the next item is under way (the query gammas and key lengths sit in
// LDS): a wait for a load issued after the stores would also wait for the stores.  The
// output goes through the V buffer that does not hold the last V tile, so the K
// buffers can take the next item's tiles meanwhile.  Each XCD owns a contiguous chunk of the items (a (batch,
// head)'s K/V stay in one L2), its W workgroups striding through the chunk; the
// batch index varies fastest over the items and W is odd, so consecutive items of a
// workgroup alternate between the samples and long and short ones spread evenly.
// ---------------------------------------------------------------------------

struct ShortItem {
  int b, h, mblk, len, ntiles;
};

__device__ __forceinline__ ShortItem short_item(const FlashArgs& a, int it, int num_m, const int* lens) {
  ShortItem r;
  r.b = it % a.B;
  const int rest = it / a.B;
  r.mblk = rest % num_m;
  r.h = rest / num_m;
  r.len = lens[r.b];
  r.ntiles = (r.len + BN - 1) / BN;
  return r;
}

// Raw query fragment of `row` (zeros past Lq) and, with the Q norm, its inverse RMS.
template <int QP>
__device__ __forceinline__ void load_q_raw(const FlashArgs& a, int b, int h, int row, int hh,
                                           bf16x8 qf[8], float& inv) {
  if (row >= a.Lq) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = bf16x8{};
    inv = 0.f;
    return;
  }
  const bf16* qp = a.q.ptr + b * a.q.sb + (int64_t)row * a.q.st + h * a.q.sh;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qp + 16 * ks + 8 * hh);
  inv = QP != kQPlain ? a.inv_rms_q[(int64_t)b * a.Lq + row] : 1.f;
}

// q' = bf16(bf16(q * inv_rms) * gamma), the reference's rounding points
// (models/fast_dit.py:145-146, 156-160).
__device__ __forceinline__ void norm_q(const bf16* gamma, int h, int hh, float inv, bf16x8 qf[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const bf16x8 g = *reinterpret_cast<const bf16x8*>(gamma + h * D + 16 * ks + 8 * hh);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bf16 t = (bf16)((float)qf[ks][j] * inv);
      qf[ks][j] = (bf16)((float)t * (float)g[j]);
    }
  }
}

// The kernel's own argument block, re-read from the kernarg segment (scalar loads,
// scalar-cache hits).  The empty asm hides the pointer's value from the compiler, so
// the fields are loaded where they are used instead of being held in SGPRs across
// the whole persistent loop (where they did not fit and were spilled).
__device__ __forceinline__ const FlashArgs& kernel_args() {
  const __attribute__((address_space(4))) char* p =
      (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *reinterpret_cast<const FlashArgs*>((const char*)p);
}

// s_waitcnt vmcnt(0) through the compiler's own builtin, so that its wait bookkeeping
// knows every earlier vector memory access has completed (expcnt and lgkmcnt fields
// at their maximum: no wait on those).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int QP>
__global__ __launch_bounds__(256, 2) void flash_short_kernel(const FlashArgs a0, int num_items) {
  constexpr int NW = 4, BM = NW * 32;
  __shared__ __attribute__((aligned(1024))) bf16 k_lds[2][kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds[2][kTileElems];
  // the query gammas (H * 128) and then the per-sample key lengths (B), copied once
  __shared__ __attribute__((aligned(16))) bf16 tab_lds[kShortTableBytes / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n32 = lane & 31, hh = lane >> 5;
  const int num_m = (a0.Lq + BM - 1) / BM;
  const int gamma_elems = QP != kQPlain ? a0.H * D : 0;
  int* const lens = reinterpret_cast<int*>(tab_lds + gamma_elems);

  // Each XCD (workgroup id % 8) owns one contiguous chunk of the items, so the
  // K/V of a (batch, head) are fetched into one XCD's L2; the W workgroups of an
  // XCD stride through its chunk.
  const int xcd = blockIdx.x % kNumXcd, per = gridDim.x / kNumXcd;
  const int base_n = num_items / kNumXcd, extra = num_items % kNumXcd;
  const int chunk_end = (xcd + 1) * base_n + min(xcd + 1, extra);
  int it = xcd * base_n + min(xcd, extra) + (int)(blockIdx.x / kNumXcd);
  if (it >= chunk_end) return;

  for (int i = tid; i < gamma_elems / 8; i += NW * 64)
    *reinterpret_cast<bf16x8*>(tab_lds + 8 * i) = *reinterpret_cast<const bf16x8*>(a0.gamma_q + 8 * i);
  for (int i = tid; i < a0.B; i += NW * 64)
    lens[i] = a0.seqlen_k != nullptr ? min(max(a0.seqlen_k[i], 0), a0.Lk) : a0.seqlen_all;
  __syncthreads();

  TileCore c;
  c.set_offsets(lane, a0.scale);
  TileLoader<NW> kl, vl;
  kl.init(a0.k.ptr, a0.k.st, wave, lane, true);
  vl.init(a0.v.ptr, a0.v.st, wave, lane, false);

  // An item's first two K tiles (global -> LDS copies into the free K buffers).
  auto prefetch_k = [&](const FlashArgs& a, const ShortItem& it) {
    if (it.ntiles > 0) {
      kl.base = reinterpret_cast<const char*>(a.k.ptr + it.b * a.k.sb + it.h * a.k.sh);
      kl.issue(0, it.len, k_lds[0], wave, lane);
      if (it.ntiles > 1) kl.issue(1, it.len, k_lds[1], wave, lane);
    }
  };

  ShortItem cur = short_item(a0, it, num_m, lens);
  float inv = 1.f;
  prefetch_k(a0, cur);
  load_q_raw<QP>(a0, cur.b, cur.h, cur.mblk * BM + wave * 32 + n32, hh, c.qf, inv);
  wait_vm_all();
  // The V buffer not holding the last V tile of the latest item with tiles: free
  // from that item's last barrier on, it stages the output.
  int vfree = 1;
  for (;;) {
    c.reset();
    if constexpr (QP != kQPlain) norm_q(tab_lds, cur.h, hh, inv, c.qf);
    const int nit = it + per;
    ShortItem nxt{};
    if (nit < chunk_end) nxt = short_item(kernel_args(), nit, num_m, lens);
    if (cur.ntiles > 0) {
      {
        const FlashArgs& a = kernel_args();
        vl.base = reinterpret_cast<const char*>(a.v.ptr + cur.b * a.v.sb + cur.h * a.v.sh);
      }
      // this item's K0 / K1 (and query rows) have landed, for every wave (each waited
      // for its own before its previous output store); every wave is done with the
      // previous item's tiles and output staging
      __syncthreads();
      vl.issue(0, cur.len, v_lds[0], wave, lane);
      f32x16 sa0, sa1, sb0, sb1;
      // V0 lands while S(0) is computed; the barrier publishes it and frees K0
      c.qk(k_lds[0], sa0, sa1);
      c.init_max(sa0, sa1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();

      auto step = [&](int t, bf16* k_fill, bf16* v_fill, const bf16* k_next, const bf16* v_cur,
                      f32x16& c0, f32x16& c1, f32x16& n0, f32x16& n1) {
        bf16x8 pb[4];
        c.finish(c0, c1, c.qk_exp(k_next, n0, n1, c0, c1, pb), pb);
        // the copies go out between the softmax and PV (3.3% faster than at the step's
        // start at lengths [470, 123]: both waves of a SIMD reach that point together)
        if (t + 2 < cur.ntiles) kl.issue(t + 2, cur.len, k_fill, wave, lane);
        vl.issue(t + 1, cur.len, v_fill, wave, lane);
        c.pv(pb, v_cur);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      };
      int t = 0;
      int vlast = 0;
      for (; t + 2 < cur.ntiles; t += 2) {
        step(t, k_lds[0], v_lds[1], k_lds[1], v_lds[0], sa0, sa1, sb0, sb1);
        step(t + 1, k_lds[1], v_lds[0], k_lds[0], v_lds[1], sb0, sb1, sa0, sa1);
      }
      if (t + 1 < cur.ntiles) {
        step(t, k_lds[0], v_lds[1], k_lds[1], v_lds[0], sa0, sa1, sb0, sb1);
        sa0 = sb0;
        sa1 = sb1;
        vlast = 1;
        ++t;
      }
      // Every wave has passed the barrier after the last S MFMAs: the K buffers
      // are free for the next item's first tiles.
      if (nit < chunk_end) {
        const FlashArgs& a = kernel_args();
        prefetch_k(a, nxt);
        load_q_raw<QP>(a, nxt.b, nxt.h, nxt.mblk * BM + wave * 32 + n32, hh, c.qf, inv);
      }
      if (cur.ntiles * BN > cur.len) c.mask_tile(sa0, sa1, t * BN, cur.len);
      bf16x8 pb[4];
      c.finish(sa0, sa1, c.exp_tile(sa0, sa1, pb), pb);
      c.pv(pb, v_lds[vlast]);
      vfree = vlast ^ 1;
    } else if (nit < chunk_end) {
      const FlashArgs& a = kernel_args();
      prefetch_k(a, nxt);
      load_q_raw<QP>(a, nxt.b, nxt.h, nxt.mblk * BM + wave * 32 + n32, hh, c.qf, inv);
    }
    // The next item's tiles and query rows were issued before this item's last tile:
    // they are waited for here, before the output stores, so that nothing after the
    // stores waits for a load issued before them (a wait for such a load would also
    // wait for the stores, which complete out of order with loads).
    wait_vm_all();
    const FlashArgs& a = kernel_args();
    c.store_out(v_lds[vfree] + wave * 2048, a.o + cur.b * a.o_sb + cur.h * a.o_sh, a.o_st,
                cur.mblk * BM + wave * 32, a.Lq, lane);
    if (nit >= chunk_end) break;
    it = nit;
    cur = nxt;
  }
}

template __global__ void flash_short_kernel<kQPlain>(const FlashArgs, int);
template __global__ void flash_short_kernel<kQNorm>(const FlashArgs, int);

// Workgroups of the persistent kernel: kNumXcd x W, W per XCD, at most two per CU
// and odd (so that one workgroup's consecutive items alternate between the samples
// of a batch of 2).
int short_grid(int items) {
  int w = 2 * (device_cu_count() / kNumXcd);
  w = w > 1 ? w - 1 : 1;
  const int need = (items + kNumXcd - 1) / kNumXcd;
  return kNumXcd * (need < w ? need : w);
}

template <int QP>
int launch_short(const FlashArgs& a, hipStream_t s) {
  const int64_t items = (int64_t)((a.Lq + 127) / 128) * a.B * a.H;
  if (items > 0x7fffffff) return set_error(2, "flash_fwd: %lld items too many", (long long)items);
  hipLaunchKernelGGL((flash_short_kernel<QP>), dim3(short_grid((int)items)), dim3(256), 0, s, a, (int)items);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "flash_fwd launch: %s", hipGetErrorString(e));
}

template <int NW, int QP>
int launch_nw(const FlashArgs& a, hipStream_t s) {
  constexpr int BM = NW * 32;
  const int64_t num_m = (a.Lq + BM - 1) / BM;
  const int64_t grid = num_m * a.B * a.H;
  if (grid > 0x7fffffff) return set_error(2, "flash_fwd: grid of %lld workgroups too large", (long long)grid);
  hipLaunchKernelGGL((flash_fwd_kernel<NW, QP>), dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "flash_fwd launch: %s", hipGetErrorString(e));
}

// Up to this many keys (the cross-attention's 512 text keys) a workgroup has 4
// waves (128 rows) and two run per CU: with only a few tiles per workgroup, one
// workgroup's start-up (Q load, first tile loads) then overlaps the other's
// tiles (measured 5% faster at 512 keys; equal or slower from 1080 keys on).
constexpr int kShortKeys = 1024;

// With per-sample key lengths the items of a short-key call differ in cost, and
// those of the short samples are mostly start-up: there the persistent kernel,
// which hides each item's start-up behind the previous item, is measured 13%
// faster (lengths 470 / 123 at Lq 7854: 87 vs 100 us).  With one key length for
// all (every item the same few tiles) the hardware's own dispatch overlaps one
// workgroup's start-up with the other's tiles as well, and the plain kernel is
// 5% faster (512 keys: 109 vs 115 us).
template <int QP>
int launch_qp(const FlashArgs& a, hipStream_t s) {
  if (a.Lk <= kShortKeys) {
    if constexpr (QP != kQNormRope) {
      // (the persistent kernel keeps the query gammas and the key lengths in LDS)
      const int table = (QP != kQPlain ? a.H * D * 2 : 0) + a.B * 4;
      if (a.seqlen_k != nullptr && table <= kShortTableBytes) return launch_short<QP>(a, s);
    }
    return launch_nw<4, QP>(a, s);
  }
  return launch_nw<kWaves, QP>(a, s);
}

}  // namespace

// CU count of the current device, queried once per device (wan_attn_init() does that
// before any launch, so that no runtime query happens inside a graph capture).
int device_cu_count() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

int launch_flash_fwd(const FlashArgs& a, hipStream_t s) {
  if (a.B == 0 || a.H == 0 || a.Lq == 0) return 0;
  switch (a.qprep) {
    case kQPlain: return launch_qp<kQPlain>(a, s);
    case kQNorm: return launch_qp<kQNorm>(a, s);
    case kQNormRope: return launch_qp<kQNormRope>(a, s);
    default: return set_error(1, "flash_fwd: unknown q preparation %d", a.qprep);
  }
}

}  // namespace wan
