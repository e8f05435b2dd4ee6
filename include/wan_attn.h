/*
 * wan_attn.h — C ABI of the MI355X (gfx950) attention path of the
 * Wan2.2-TI2V-5B DiT: flash self-attention, cross-attention with per-sample
 * key lengths, QK-RMSNorm and 3D-RoPE (standalone and fused into the
 * attention kernels).
 *
 * Conventions
 *   - Tensors are bf16 device pointers in the DiT projection layout
 *     [batch, token, head, head_dim] (a view of [batch, token, dim]) described
 *     by wan_tensor: element strides of batch, token and head; head_dim is
 *     contiguous.  head_dim must be 128, the data pointer 16-byte aligned and
 *     every stride a multiple of 8 elements.
 *   - RoPE tables are fp32 [seqlen, head_dim/2] cos and sin (the layout of
 *     _rope_tables, models/fast_dit.py:548-558, without the unit dims).
 *   - Outputs and workspaces are allocated by the caller; the library never
 *     allocates or frees device memory and never synchronises the stream.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Every call is
 *     asynchronous and re-entrant.
 *   - softmax_scale (every attention entry point) must be finite and > 0; other
 *     values return WAN_ERR_UNSUPPORTED.
 *   - Return value: WAN_OK or an error code; wan_attn_last_error() returns the
 *     calling thread's last message.
 */
#ifndef WAN_ATTN_H
#define WAN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum wan_status {
  WAN_OK = 0,
  WAN_ERR_INVALID = 1,     /* bad pointer, shape, stride or length */
  WAN_ERR_UNSUPPORTED = 2, /* valid but outside what the kernels implement (head_dim != 128, ...) */
  WAN_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  WAN_ERR_LAUNCH = 4       /* the HIP runtime rejected a launch */
};

/* A [batch, token, head, head_dim] bf16 device tensor. */
typedef struct wan_tensor {
  void* data;
  int64_t batch_stride;
  int64_t token_stride;
  int64_t head_stride;
} wan_tensor;

/* Message of the calling thread's last failed call ("" if none). */
const char* wan_attn_last_error(void);

/* ABI version of this header (incremented on incompatible changes). */
int wan_attn_abi_version(void);

/*
 * Set-up for the current device: looks up the device address of the library's static
 * scratch (used by wan_cross_attn_fused_noalloc) once, so that no runtime lookup happens
 * later inside a HIP graph capture.  Idempotent; call it with each device current that
 * will run the no-allocation entry point.  Allocates nothing.  No counterpart in the
 * reference (its kernels have no library-owned device state).
 */
int wan_attn_init(void);

/*
 * Self-attention, out = softmax(q k^T * softmax_scale) v over the first
 * actual_seqlen_k keys (actual_seqlen_k <= 0 means all seqlen_k keys).
 * Replaces wan_flash_self_attn, kernels/self_attention_nst.py:49-117, and the
 * _sdpa / _nki_self backends, models/fast_dit.py:186-207, without their
 * permute/pad copies: q [B, Lq, H, 128], k/v [B, Lk, H, 128] -> out [B, Lq, H, 128].
 */
int wan_flash_self_attn(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                        int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                        float softmax_scale, int actual_seqlen_k, void* stream);

/*
 * Cross-attention over text keys with per-sample key lengths:
 * out[b] = softmax(q[b] k[b, :len_b]^T * scale) v[b, :len_b], len_b =
 * seqlen_k_dev[b] (device int32 [batch], clamped to [0, seqlen_k]; a sample
 * with len 0 gets zeros).  seqlen_k_dev == NULL attends to all seqlen_k keys,
 * as the reference kernel does.
 * Replaces wan_cross_attn, kernels/cross_attention.py:17-123, and _nki_cross,
 * models/fast_dit.py:244-255.
 */
int wan_cross_attn(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                   int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                   float softmax_scale, const int32_t* seqlen_k_dev, void* stream);

/*
 * Fused self-attention span of _FastBlock.forward, models/fast_dit.py:281-292:
 *   q,k = _tp_rms_qk(q, k) (RMS over all heads*128 channels of a token, eps,
 *         bf16 gamma [heads*128]); q,k = _rope(q), _rope(k); out = attention(q, k, v).
 * q, k, v are the raw projections [B, L, H, 128].  The per-token RMS of q and
 * the normalised, rotated k are written to `workspace` (at least
 * wan_self_attn_fused_workspace() bytes, 256-byte aligned); q is normalised
 * and rotated inside the attention kernel as it is loaded.
 */
size_t wan_self_attn_fused_workspace(int batch, int heads, int seqlen);
int wan_self_attn_fused(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                        int batch, int heads, int seqlen, int head_dim,
                        const void* gamma_q, const void* gamma_k, float eps,
                        const float* rope_cos, const float* rope_sin, float softmax_scale,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused cross-attention span, models/fast_dit.py:297-304:
 *   q = _tp_rms(q, norm_q); out = cross attention(q, k, v) with per-sample key
 * lengths as wan_cross_attn.  k is the per-prompt normalised cross K
 * (_FastCrossKV, models/fast_dit.py:464-477).  Workspace holds the per-token
 * RMS of q (at least wan_cross_attn_fused_workspace() bytes).
 */
size_t wan_cross_attn_fused_workspace(int batch, int heads, int seqlen_q);
int wan_cross_attn_fused(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                         int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                         const void* gamma_q, float eps, float softmax_scale,
                         const int32_t* seqlen_k_dev,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * wan_cross_attn_fused without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The per-row inverse RMS of q goes
 * to a scratch array owned by the library: WAN_NOALLOC_MAX_ROWS fp32 rows (512 KB) per
 * GPU, held until the process ends; batch * seqlen_q above that returns
 * WAN_ERR_UNSUPPORTED.  The array's device address is looked up by wan_attn_init() on
 * the device current at that call; without it, on the entry point's first call on each
 * device.  A caller that captures the first call into a HIP graph calls wan_attn_init()
 * on that device before the capture begins.  Nothing is allocated or freed.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (e.g. on two
 * streams) race and must be ordered by the caller.  Same kernels and results as
 * wan_cross_attn_fused.
 */
#define WAN_NOALLOC_MAX_ROWS (1 << 17)
int wan_cross_attn_fused_noalloc(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                                 int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                                 const void* gamma_q, float eps, float softmax_scale,
                                 const int32_t* seqlen_k_dev, void* stream);

/*
 * 3D-RoPE interleaved-pair rotation in fp32 with one bf16 rounding:
 * out [B, L, H, 128] contiguous.  Semantics of _rope, models/fast_dit.py:163-169
 * (the named kernel causal_rope_rotation, kernels/rope.py:39-71, computes the
 * same rotation from an expanded cos / signed-sin table).
 */
int wan_rope(wan_tensor x, void* out, int batch, int seqlen, int heads, int head_dim,
             const float* rope_cos, const float* rope_sin, void* stream);

/*
 * RMSNorm over all heads*128 channels of each token with bf16 gamma, the
 * reference's rounding, optionally followed by the 3D-RoPE rotation:
 *   out = rope(bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gamma))
 * _tp_rms at TP=1, models/fast_dit.py:156-160 (on q and k it is _tp_rms_qk,
 * :134-147; with rope_cos/rope_sin it is the K side of :281-284).  out:
 * [B, L, H, 128] contiguous, may be NULL when only inv_rms_out (fp32 [B*L],
 * may be NULL) is wanted; rope_cos/rope_sin may be NULL (no rotation).
 */
int wan_rms_norm(wan_tensor x, void* out, int batch, int seqlen, int heads, int head_dim,
                 const void* gamma, float eps, const float* rope_cos, const float* rope_sin,
                 float* inv_rms_out, void* stream);

/*
 * The two RMSNorm passes of a fused self-attention in one launch, as
 * _tp_rms_qk treats q and k together (models/fast_dit.py:134-147, TP=1):
 * inv_rms_q (fp32 [B*L]) = 1/rms of each q token over heads*128 channels, and
 * k_out ([B, L, H, 128] contiguous) = rope(bf16(bf16(k * inv_rms_k) * gamma_k))
 * as wan_rms_norm computes it (rope_cos/rope_sin NULL: no rotation).
 */
int wan_rms_norm_qk(wan_tensor q, wan_tensor k, void* k_out, int batch, int seqlen, int heads,
                    int head_dim, const void* gamma_k, float eps, const float* rope_cos,
                    const float* rope_sin, float* inv_rms_q, void* stream);

/*
 * wan_rms_norm_qk with the sums of squares taken from wan_qkv_proj_sumsq instead of the
 * rows (models/fast_dit.py:134-147 with the statistics from the projection's epilogue):
 * sumsq fp32 [4 * heads, B * L], the GEMM's 64-column partials of q (rows 0 .. 2 heads - 1)
 * and k (2 heads .. 4 heads - 1) for every token (GEMM row b * L + l).  Writes inv_rms_q
 * (fp32 [B*L]) without reading q, and k_out = rope(bf16(bf16(k * inv_rms_k) * gamma_k)).
 */
int wan_rms_norm_qk_sumsq(wan_tensor k, void* k_out, int batch, int seqlen, int heads, int head_dim,
                          const void* gamma_k, float eps, const float* rope_cos, const float* rope_sin,
                          const float* sumsq, float* inv_rms_q, void* stream);

/*
 * Attention whose query is normalised inside the kernel as it is loaded:
 *   q' = rope?(bf16(bf16(q * inv_rms_q[b, i]) * gamma_q)),  out = softmax(q' k^T * scale) v
 * with inv_rms_q from wan_rms_norm (fp32 [B*Lq]).  rope_cos/rope_sin NULL: no
 * rotation (the cross-attention query, models/fast_dit.py:297-298); non-NULL:
 * the self-attention query (:281-283), tables of seqlen_q rows.  seqlen_k_dev
 * as in wan_cross_attn.  This is the kernel behind the two fused entry points.
 */
int wan_flash_attn_qnorm(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                         int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                         const float* inv_rms_q, const void* gamma_q,
                         const float* rope_cos, const float* rope_sin, float softmax_scale,
                         const int32_t* seqlen_k_dev, void* stream);

/*
 * One adaLN stage of a WanAttentionBlock (the pointwise work between its
 * GEMMs), fused into one pass over the residual stream.  With f the frame of
 * the token (seqlen / frames contiguous tokens per frame) and e[f, i] the
 * modulation rows:
 *   r     = x | bf16(x + y) | bf16(x + bf16(y * e[f, gate_idx]))
 *   x_out = r                                       (written when non-NULL)
 *   ln    = bf16(LayerNorm(r) [* ln_weight + ln_bias])   fp32 statistics, eps
 *   h_out = ln | bf16(bf16(ln * bf16(1 + e[f, scale_idx])) + e[f, shift_idx])
 * Replaces the eager ops of models/fast_dit.py:280 (norm1 + _modulate), :294
 * (x + _gate(y) then norm3), :306-307 (x + cross output, norm2 + _modulate) and
 * :311 (x + _gate(y)); _modulate / _gate are :172-181, WanLayerNorm is
 * wan/modules/model.py:89-99.  x, y, x_out, h_out: [batch, seqlen, dim] bf16
 * contiguous; e: [frames, 6, dim] bf16 contiguous (block modulation + time
 * projection, models/fast_dit.py:275-276); indices -1 = absent.  y, x_out,
 * h_out, e, ln_weight/ln_bias may be NULL as the stage needs.
 */
int wan_adaln(const void* x, const void* y, void* x_out, void* h_out, int batch, int seqlen,
              int dim, const void* e, int frames, int gate_idx, int shift_idx, int scale_idx,
              const void* ln_weight, const void* ln_bias, float eps, void* stream);

/*
 * wan_adaln with the shift and scale rows taken from another row set, e_mod
 * [frames, mod_rows, dim] (mod_rows in 1..6), while the gate keeps e's rows:
 *   h_out = ln | bf16(bf16(ln * bf16(1 + e_mod[f, scale_idx])) + e_mod[f, shift_idx])
 * One pass then ends one block and starts the next: the gated residual of block i
 * (models/fast_dit.py:311, gate e_i[f, 5]) followed by block i+1's norm1 + _modulate
 * (:280, rows e_{i+1}[f, 0..1]); or, after the last block, the output head's LayerNorm
 * and modulation (models/fast_dit.py:480-505: two rows per frame, mod_rows = 2).
 * The results are those of the two separate stages bit for bit (the residual is
 * rounded to bf16 before its LayerNorm statistics, as when re-read).  e_mod = NULL is
 * wan_adaln.  No counterpart of its own in the reference: it fuses two of its stages.
 */
int wan_adaln_ex(const void* x, const void* y, void* x_out, void* h_out, int batch, int seqlen,
                 int dim, const void* e, int frames, int gate_idx, const void* e_mod, int mod_rows,
                 int shift_idx, int scale_idx, const void* ln_weight, const void* ln_bias, float eps,
                 void* stream);

/*
 * The block's q/k/v projection with the statistics of the QK-RMSNorm in its epilogue:
 *   out[m, n]   = bf16(sum_k x[m, k] w[n, k] + bias[n])           (bf16, fp32 accumulation)
 *   sumsq[p, m] = sum over columns 64 p .. 64 p + 63 of bf16(out[m, n])^2,  p < sq_cols / 64
 * x [M, K] (row stride ldx), w [N, K] (ldw; an nn.Linear weight: the concatenated q, k, v
 * weights), bias [N], out [M, N] (ldo), sumsq fp32 [sq_cols / 64, M].  Replaces
 * _lin(h, sa.q), _lin(h, sa.k), _lin(h, sa.v) of models/fast_dit.py:281-282 together with
 * the per-token sums of squares of _tp_rms_qk (:134-147): with sq_cols = 2 * heads * 128
 * the q and k sums of every head come out of the GEMM and wan_self_attn_fused_sumsq needs
 * no q statistics pass.  N must be a multiple of 256, K of 64, sq_cols of 64.
 */
int wan_qkv_proj_sumsq(const void* x, const void* w, const void* bias, void* out, float* sumsq,
                       int M, int N, int K, int64_t ldx, int64_t ldw, int64_t ldo, int sq_cols,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WAN_ATTN_H */
