// The block's q/k/v projection as one bf16 GEMM on gfx950, with the statistics of the
// QK-RMSNorm in its epilogue:
//
//   out[m, n]    = bf16(sum_k x[m, k] w[n, k] + bias[n])          (F.linear, models/fast_dit.py:281)
//   sumsq[p, m]  = sum over columns 64 p .. 64 p + 63 of bf16(out[m, n])^2,  for 64 p < sq_cols
//
// so that the per-token sums of squares of q and k over all heads (_tp_rms_qk,
// models/fast_dit.py:134-147) are 48 + 48 partial sums read by the K pass, and q is
// not read again before the attention kernel.
//
// Design: 256 x 256 output tile per workgroup, 8 waves in a 2 x 4 grid, each wave
// 128 (m) x 64 (n): 8 accumulators of v_mfma_f32_32x32x16_bf16, two waves per SIMD.
// The MFMA computes out^T tiles, w rows on the MFMA row axis and x rows on the column
// axis, so a lane holds one output row (lane % 32) and half of each 64-column block: a
// 64-column sum of squares is lane-local plus one exchange with the lane 32 apart, as
// the attention kernel's softmax row sums are.  K advances 64 per tile; the 256 x 64
// tiles of x and w (32 KB each) go global -> LDS by 16-byte copies into rows of eight
// 16-byte chunks, chunk c of row r at position c ^ ((r / 2) % 8) (conflict-free operand
// reads), in two slots, one barrier per tile.  Program order is pinned MFMA by MFMA:
// each MFMA is followed by one fragment read of the next k-step and, in a tile's first
// k-step, one copy of the next tile, and the barrier sits inside the last k-step so the
// next tile's first reads overlap its remaining MFMAs.  Workgroups run in groups of 8
// M-tiles per N-tile, each XCD owning a contiguous range, so the tiles running together
// on an XCD share x and w rows in its L2.
//
// At the QKV shape (M 15708, N 9216, K 3072) it reaches 1.28-1.31 PFLOP/s, 86-88% of
// hipBLASLt's F.linear timed beside it, with output bit-identical.  Both are power
// limited (all-zero operands run either ~25% faster); on zeros this kernel's k-loop is
// ~13% slower per tile than hipBLASLt's.  4 waves of 128 x 128 (a third less LDS read
// traffic, one wave per SIMD) run the loop at a higher clock (1.72 vs 1.58 GHz) but in
// more cycles per tile, and tie with this tiling at best.
#include "launchers.h"

#include <type_traits>

namespace wan {

namespace {

constexpr int GBM = 256, GBN = 256;
constexpr int kGroupM = 8;
// 8 waves in a 2 x 4 grid (each 128 x 64 of the 256 x 256 tile, two waves per SIMD),
// 64 k per stage: measured the fastest of 2 x 2 / 2 x 4 waves, 32 / 64 k, 2-5 stages
constexpr int kGemmWM = 2, kGemmWN = 4, kGemmBK = 64;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t lds_addr(const bf16* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) bf16*)p;
}

// 16-byte global -> LDS copy (lane l writes LDS bytes m0 + 16 l ..), from inline asm so
// the compiler's LDS wait counting does not see it (see flash_fwd.hip); completion is
// waited for explicitly before the barrier that publishes a stage.  A memory instruction
// needs 5 wait states after a VALU write (v_readfirstlane / v_readlane) of an SGPR it
// reads, and the compiler does not pad that for inline asm: the scalar base of this copy
// and of flash_fwd.hip's must come from scalar code (tests/test_isa_hazards.py checks
// the compiled kernels).
__device__ __forceinline__ void dma16(const char* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int WM, int WN, int BK>
struct GemmCfg {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TM = GBM / WM / 32;        // 32-row blocks of x (output rows) per wave
  static constexpr int TN = GBN / WN / 32;        // 32-row blocks of w (output columns) per wave
  static constexpr int kCpr = BK / 8;             // 16-byte chunks per tile row
  static constexpr int kRps = 16 / kCpr;          // rows per 256-byte bank sweep
  static constexpr int kTileElems = 256 * BK;
  static constexpr int kBlocks = kTileElems / 512; // 1 KB copies per tile
  static constexpr int kPerWave = kBlocks / kWaves;
  static constexpr int kRowsPerBlock = 512 / BK;  // tile rows per 1 KB copy
  static_assert(kBlocks % kWaves == 0, "copies must divide over the waves");
  // chunk c of row r sits at position c ^ ((r / kRps) % kCpr): the 16 rows read by a
  // 16-lane phase of an operand read land on 16 distinct 16-byte bank groups
  __device__ static __forceinline__ int swz(int row) { return (row / kRps) & (kCpr - 1); }
};

// Copies of one 256 x BK tile in 1 KB blocks, wave w issuing blocks w, w + waves, ...
// Lane l fills LDS row (block rows) + l / kCpr, position l % kCpr, with the global chunk
// the row's swizzle puts there.  Offsets are bytes from the tile's (row 0, k 0).
template <class C>
struct GemmTileLoader {
  uint32_t off[C::kPerWave];
  __device__ void init(int64_t ld, int rows_valid, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < C::kPerWave; ++i) {
      const int row = C::kRowsPerBlock * (wave + C::kWaves * i) + lane / C::kCpr;
      const int r = min(row, rows_valid - 1);       // rows past the matrix repeat its last row
      off[i] = (uint32_t)((int64_t)r * ld * 2 + (((lane % C::kCpr) ^ C::swz(row)) << 4));
    }
  }
  __device__ __forceinline__ void issue(const char* tile_base, bf16* dst, int wave) const {
#pragma unroll
    for (int i = 0; i < C::kPerWave; ++i) issue_one(tile_base, dst, wave, i);
  }
  __device__ __forceinline__ void issue_one(const char* tile_base, bf16* dst, int wave, int i) const {
    dma16(tile_base, off[i], lds_addr(dst + (wave + C::kWaves * i) * 512));
  }
};

template <int WM, int WN, int BK>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_rowsq_kernel(const GemmArgs a) {
  using C = GemmCfg<WM, WN, BK>;
  __shared__ __attribute__((aligned(1024))) bf16 xs[2][C::kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 ws[2][C::kTileElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int l32 = lane & 31, hh = lane >> 5;

  // tile order: groups of kGroupM M-tiles, N-tiles within a group, each XCD a range
  const int mt_count = (a.M + GBM - 1) / GBM, nt_count = a.N / GBN;
  const int pid = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = kGroupM * nt_count;
  const int group = pid / per_group, first_m = group * kGroupM;
  const int gsize = min(mt_count - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  const int tm = first_m + in_group % gsize, tn = in_group / gsize;
  const int m0 = tm * GBM, n0 = tn * GBN;

  GemmTileLoader<C> xl, wl;
  xl.init(a.ldx, a.M - m0, wave, lane);
  wl.init(a.ldw, GBN, wave, lane);
  const char* xbase = reinterpret_cast<const char*>(a.x + (int64_t)m0 * a.ldx);
  const char* wbase = reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw);

  // operand rows of this lane within the tiles; (row / kRps) % kCpr is the same for
  // every 32-row block
  int xrow[C::TM], wrow[C::TN];
#pragma unroll
  for (int b = 0; b < C::TM; ++b) xrow[b] = (wm * C::TM + b) * 32 + l32;
#pragma unroll
  for (int b = 0; b < C::TN; ++b) wrow[b] = (wn * C::TN + b) * 32 + l32;
  const int sw = C::swz(l32);

  // the bias of this wave's columns, loaded before the k-loop: in the epilogue its
  // loads stood first on the critical path (1-1.3% of the launch)
  constexpr int kCols = C::TN * 32;              // this wave's columns (64 or 128)
  bf16x4 bias_r[C::TN][4];
#pragma unroll
  for (int nb = 0; nb < C::TN; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      bias_r[nb][g] = *reinterpret_cast<const bf16x4*>(a.bias + n0 + wn * kCols + nb * 32 + 8 * g + 4 * hh);

  f32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
#pragma unroll
    for (int j = 0; j < C::TM; ++j) acc[i][j] = f32x16{};

  const int kt_count = a.K / BK;
  auto read_frag = [&](int slot, int ks, int i, bf16x8 wf[C::TN], bf16x8 xf[C::TM]) {
    const int pos = ((2 * ks + hh) ^ sw) << 3;
    if (i < C::TN)
      wf[i] = *reinterpret_cast<const bf16x8*>(ws[slot] + wrow[i] * BK + pos);
    else
      xf[i - C::TN] = *reinterpret_cast<const bf16x8*>(xs[slot] + xrow[i - C::TN] * BK + pos);
  };
  auto copy_one = [&](int slot, int kt, int i) {
    const int64_t kb = (int64_t)kt * BK * 2;
    if (i < C::kPerWave)
      xl.issue_one(xbase + kb, xs[slot], wave, i);
    else
      wl.issue_one(wbase + kb, ws[slot], wave, i - C::kPerWave);
  };
  constexpr int KS = BK / 16;             // MFMA k-steps per tile
  constexpr int NF = C::TN + C::TM;       // fragment reads per k-step
  constexpr int NM = C::TN * C::TM;       // MFMAs per k-step
  constexpr int NC = 2 * C::kPerWave;     // copies per tile and wave
  constexpr int SPLIT = NM - NF;          // MFMAs of the last k-step before the barrier
  static_assert(KS % 2 == 0 && NF <= NM, "schedule");

  bf16x8 wf[2][C::TN], xf[2][C::TM];

  // One tile of k.  Program order is fixed MFMA by MFMA (a scheduling barrier after
  // each): after MFMA m of k-step ks comes fragment read m of k-step ks + 1 (the reads
  // are in flight behind the MFMAs that follow) and, in k-step 0, copy m of the next
  // tile into the other slot.  The last k-step splits around the barrier that publishes
  // the next tile: NM - NF MFMAs, the copies' wait and the barrier, then NF MFMAs, each
  // followed by a read of the next tile's first k-step.
  auto tile = [&](int kt, auto has_next_c) {
    constexpr bool has_next = decltype(has_next_c)::value;
    const int slot = kt & 1, nslot = slot ^ 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (ks == KS - 1 && m == SPLIT) {
          // every wave's copies of the next tile landed, every read of this slot returned
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
          __builtin_amdgcn_sched_barrier(0);
        }
        const int nb = m / C::TM, mb = m % C::TM;
        acc[nb][mb] = mfma32(wf[cur][nb], xf[cur][mb], acc[nb][mb]);
        if (ks < KS - 1) {
          if (m < NF) read_frag(slot, ks + 1, m, wf[nxt], xf[nxt]);
        } else if (has_next && m >= SPLIT) {
          read_frag(nslot, 0, m - SPLIT, wf[nxt], xf[nxt]);
        }
        if (has_next && ks == 0 && m < NC) copy_one(nslot, kt + 1, m);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (has_next && ks == 0) {
#pragma unroll
        for (int i = NM; i < NC; ++i) copy_one(nslot, kt + 1, i);
      }
    }
  };

  for (int i = 0; i < NC; ++i) copy_one(0, 0, i);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NF; ++i) read_frag(0, 0, i, wf[0], xf[0]);
  for (int kt = 0; kt + 1 < kt_count; ++kt) tile(kt, std::integral_constant<bool, true>{});
  tile(kt_count - 1, std::integral_constant<bool, false>{});
  __syncthreads();   // every wave is done with the last stage before the output staging

  // Epilogue, one 32-row block at a time: bias, bf16 rounding, the sums of squares over
  // each 64 of this wave's columns, then the block staged through this wave's LDS
  // (row-major, chunk c of row r at position c ^ (r % chunks)) and stored as whole row
  // segments.
  constexpr int kChunks = kCols / 8;
  bf16* stage = &xs[0][0] + wave * 32 * kCols;
  const int ncol0 = n0 + wn * kCols;
#pragma unroll
  for (int mb = 0; mb < C::TM; ++mb) {
    const int row0 = m0 + (wm * C::TM + mb) * 32;
    float ss[C::TN / 2] = {};   // per 64 columns (two 32-column blocks)
#pragma unroll
    for (int nb = 0; nb < C::TN; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const bf16x4 b4 = bias_r[nb][g];
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (bf16)(acc[nb][mb][4 * g + e] + (float)b4[e]);
          const float f = (float)v[e];
          ss[nb / 2] = fmaf(f, f, ss[nb / 2]);
        }
        const int c = 4 * nb + g;   // this lane's columns 8c + 4hh .. +3 of row l32
        *reinterpret_cast<bf16x4*>(stage + l32 * kCols + ((c ^ (l32 % kChunks)) << 3) + 4 * hh) = v;
      }
    }
#pragma unroll
    for (int h = 0; h < C::TN / 2; ++h) {
      const float t = pair_sum(ss[h]);
      if (ncol0 + 64 * h < a.sq_cols && hh == 0 && row0 + l32 < a.M)
        a.sumsq[(int64_t)(ncol0 / 64 + h) * a.M + row0 + l32] = t;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    constexpr int kRowsPerStore = 64 / kChunks;
#pragma unroll
    for (int j = 0; j < 32 / kRowsPerStore; ++j) {
      const int r = kRowsPerStore * j + lane / kChunks, c = lane % kChunks;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(stage + r * kCols + ((c ^ (r % kChunks)) << 3));
      if (row0 + r < a.M)
        __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(a.out + (int64_t)(row0 + r) * a.ldo + ncol0 + 8 * c));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

}  // namespace

int launch_gemm_rowsq(const GemmArgs& a, hipStream_t s) {
  if (a.M == 0) return 0;
  const int64_t tiles = (int64_t)((a.M + GBM - 1) / GBM) * (a.N / GBN);
  if (tiles > 0x7fffffff) return set_error(2, "gemm: %lld tiles too many", (long long)tiles);
  hipLaunchKernelGGL((gemm_rowsq_kernel<kGemmWM, kGemmWN, kGemmBK>), dim3((unsigned)tiles),
                     dim3(64 * kGemmWM * kGemmWN), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : set_error(4, "gemm launch: %s", hipGetErrorString(e));
}

}  // namespace wan
