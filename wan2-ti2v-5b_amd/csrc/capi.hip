// C-ABI entry points (include/wan_attn.h): argument validation, workspace
// layout and dispatch to the kernels.  Nothing here allocates device memory
// or synchronises the stream.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/wan_attn.h"
#include "launchers.h"

namespace wan {

namespace {
thread_local char g_last_error[512] = "";

constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

Tensor4 as_t4(const wan_tensor& t) {
  return Tensor4{static_cast<const bf16*>(t.data), t.batch_stride, t.token_stride, t.head_stride};
}

// Checks one [B, L, H, 128] operand: pointer, alignment, stride granularity.
int check_tensor(const char* fn, const char* name, const wan_tensor& t, int B, int L, int H) {
  if (B > 0 && L > 0 && H > 0 && t.data == nullptr)
    return set_error(WAN_ERR_INVALID, "%s: %s is NULL", fn, name);
  if (reinterpret_cast<uintptr_t>(t.data) % 16 != 0)
    return set_error(WAN_ERR_INVALID, "%s: %s is not 16-byte aligned", fn, name);
  if (t.batch_stride % 8 || t.token_stride % 8 || t.head_stride % 8)
    return set_error(WAN_ERR_INVALID,
                     "%s: %s strides (%lld, %lld, %lld) must be multiples of 8 elements", fn, name,
                     (long long)t.batch_stride, (long long)t.token_stride, (long long)t.head_stride);
  if (t.batch_stride < 0 || t.token_stride < 0 || t.head_stride < 0)
    return set_error(WAN_ERR_INVALID, "%s: %s has a negative stride", fn, name);
  // the attention tile loads keep row * token_stride of a 64-key tile in 32-bit byte offsets
  if (t.token_stride >= (int64_t(1) << 24))
    return set_error(WAN_ERR_UNSUPPORTED, "%s: %s token stride %lld exceeds 2^24 elements", fn, name,
                     (long long)t.token_stride);
  return WAN_OK;
}

int check_dims(const char* fn, int B, int H, int Lq, int Lk, int D) {
  if (B < 0 || H < 0 || Lq < 0 || Lk < 0)
    return set_error(WAN_ERR_INVALID, "%s: negative size (B=%d H=%d Lq=%d Lk=%d)", fn, B, H, Lq, Lk);
  if (D != kHeadDim)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: head_dim=%d, only 128 is implemented", fn, D);
  if (H * kHeadDim > 8192)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: heads*128=%d exceeds 8192 channels", fn, H * kHeadDim);
  return WAN_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// The kernels scale scores by softmax_scale * log2(e) and rely on that factor being
// finite and positive (masked keys are -inf, the running max is a max of scaled scores).
int check_scale(const char* fn, float scale) {
  if (!(scale > 0.f) || !(scale < INFINITY))
    return set_error(WAN_ERR_UNSUPPORTED, "%s: softmax_scale=%g, must be finite and > 0", fn, (double)scale);
  return WAN_OK;
}

// Validates the arguments of one RMSNorm / statistics task and fills its PrepArgs.
int rms_prep_args(const char* fn, wan_tensor x, void* out, int batch, int seqlen, int heads,
                  int head_dim, const void* gamma, float eps, const float* rope_cos,
                  const float* rope_sin, float* inv_rms_out, PrepArgs* a) {
  int rc;
  if ((rc = check_dims(fn, batch, heads, seqlen, seqlen, head_dim))) return rc;
  if ((rc = check_tensor(fn, "x", x, batch, seqlen, heads))) return rc;
  if (out && !aligned16(out)) return set_error(WAN_ERR_INVALID, "%s: out must be 16-byte aligned", fn);
  if (out && (!gamma || !aligned16(gamma)))
    return set_error(WAN_ERR_INVALID, "%s: gamma must be a 16-byte aligned pointer", fn);
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: rope_cos and rope_sin must both be given or both NULL", fn);
  if (rope_cos && (!out || !aligned16(rope_cos) || !aligned16(rope_sin)))
    return set_error(WAN_ERR_INVALID, "%s: rotation needs `out` and 16-byte aligned tables", fn);
  if (!(eps >= 0.f)) return set_error(WAN_ERR_INVALID, "%s: eps must be >= 0", fn);
  a->x = as_t4(x);
  a->B = batch;
  a->L = seqlen;
  a->H = heads;
  a->eps = eps;
  a->inv_rms = inv_rms_out;
  a->gamma = static_cast<const bf16*>(gamma);
  a->cos = rope_cos;
  a->sin = rope_sin;
  a->out = static_cast<bf16*>(out);
  return WAN_OK;
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace wan

using namespace wan;

extern "C" {

const char* wan_attn_last_error(void) { return g_last_error; }

int wan_attn_abi_version(void) { return 1; }

int wan_flash_self_attn(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out, int batch,
                        int heads, int seqlen_q, int seqlen_k, int head_dim, float softmax_scale,
                        int actual_seqlen_k, void* stream) {
  const char* fn = "wan_flash_self_attn";
  int rc;
  if ((rc = check_scale(fn, softmax_scale))) return rc;
  if ((rc = check_dims(fn, batch, heads, seqlen_q, seqlen_k, head_dim))) return rc;
  if ((rc = check_tensor(fn, "q", q, batch, seqlen_q, heads))) return rc;
  if ((rc = check_tensor(fn, "k", k, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "v", v, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "out", out, batch, seqlen_q, heads))) return rc;
  if (actual_seqlen_k <= 0) actual_seqlen_k = seqlen_k;
  if (actual_seqlen_k > seqlen_k)
    return set_error(WAN_ERR_INVALID, "%s: actual_seqlen_k=%d exceeds seqlen_k=%d", fn,
                     actual_seqlen_k, seqlen_k);
  if (seqlen_q > 0 && seqlen_k == 0)
    return set_error(WAN_ERR_INVALID, "%s: no keys (seqlen_k=0)", fn);
  FlashArgs a{};
  a.q = as_t4(q);
  a.k = as_t4(k);
  a.v = as_t4(v);
  a.o = static_cast<bf16*>(out.data);
  a.o_sb = out.batch_stride;
  a.o_st = out.token_stride;
  a.o_sh = out.head_stride;
  a.B = batch;
  a.H = heads;
  a.Lq = seqlen_q;
  a.Lk = seqlen_k;
  a.seqlen_k = nullptr;
  a.seqlen_all = actual_seqlen_k;
  a.scale = softmax_scale;
  a.qprep = kQPlain;
  return launch_flash_fwd(a, static_cast<hipStream_t>(stream));
}

int wan_cross_attn(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out, int batch, int heads,
                   int seqlen_q, int seqlen_k, int head_dim, float softmax_scale,
                   const int32_t* seqlen_k_dev, void* stream) {
  const char* fn = "wan_cross_attn";
  int rc;
  if ((rc = check_scale(fn, softmax_scale))) return rc;
  if ((rc = check_dims(fn, batch, heads, seqlen_q, seqlen_k, head_dim))) return rc;
  if ((rc = check_tensor(fn, "q", q, batch, seqlen_q, heads))) return rc;
  if ((rc = check_tensor(fn, "k", k, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "v", v, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "out", out, batch, seqlen_q, heads))) return rc;
  FlashArgs a{};
  a.q = as_t4(q);
  a.k = as_t4(k);
  a.v = as_t4(v);
  a.o = static_cast<bf16*>(out.data);
  a.o_sb = out.batch_stride;
  a.o_st = out.token_stride;
  a.o_sh = out.head_stride;
  a.B = batch;
  a.H = heads;
  a.Lq = seqlen_q;
  a.Lk = seqlen_k;
  a.seqlen_k = seqlen_k_dev;
  a.seqlen_all = seqlen_k;
  a.scale = softmax_scale;
  a.qprep = kQPlain;
  return launch_flash_fwd(a, static_cast<hipStream_t>(stream));
}

size_t wan_self_attn_fused_workspace(int batch, int heads, int seqlen) {
  if (batch <= 0 || heads <= 0 || seqlen <= 0) return 0;
  const size_t rows = (size_t)batch * seqlen;
  return align_up(rows * sizeof(float)) + align_up(rows * heads * kHeadDim * sizeof(bf16));
}

int wan_rms_norm(wan_tensor x, void* out, int batch, int seqlen, int heads, int head_dim,
                 const void* gamma, float eps, const float* rope_cos, const float* rope_sin,
                 float* inv_rms_out, void* stream) {
  PrepArgs a{};
  int rc;
  if ((rc = rms_prep_args("wan_rms_norm", x, out, batch, seqlen, heads, head_dim, gamma, eps,
                          rope_cos, rope_sin, inv_rms_out, &a)))
    return rc;
  if ((int64_t)batch * seqlen * heads == 0) return WAN_OK;
  return launch_rms_prep(a, static_cast<hipStream_t>(stream));
}

int wan_rms_norm_qk(wan_tensor q, wan_tensor k, void* k_out, int batch, int seqlen, int heads,
                    int head_dim, const void* gamma_k, float eps, const float* rope_cos,
                    const float* rope_sin, float* inv_rms_q, void* stream) {
  const char* fn = "wan_rms_norm_qk";
  if (inv_rms_q == nullptr || k_out == nullptr)
    return set_error(WAN_ERR_INVALID, "%s: inv_rms_q and k_out are required", fn);
  PrepArgs aq{}, ak{};
  int rc;
  if ((rc = rms_prep_args(fn, q, nullptr, batch, seqlen, heads, head_dim, nullptr, eps, nullptr,
                          nullptr, inv_rms_q, &aq)))
    return rc;
  if ((rc = rms_prep_args(fn, k, k_out, batch, seqlen, heads, head_dim, gamma_k, eps, rope_cos,
                          rope_sin, nullptr, &ak)))
    return rc;
  if ((int64_t)batch * seqlen * heads == 0) return WAN_OK;
  return launch_rms_prep2(aq, ak, static_cast<hipStream_t>(stream));
}

int wan_rms_norm_qk_sumsq(wan_tensor k, void* k_out, int batch, int seqlen, int heads, int head_dim,
                          const void* gamma_k, float eps, const float* rope_cos, const float* rope_sin,
                          const float* sumsq, float* inv_rms_q, void* stream) {
  const char* fn = "wan_rms_norm_qk_sumsq";
  if (inv_rms_q == nullptr || k_out == nullptr || sumsq == nullptr)
    return set_error(WAN_ERR_INVALID, "%s: sumsq, inv_rms_q and k_out are required", fn);
  if (!aligned16(sumsq)) return set_error(WAN_ERR_INVALID, "%s: sumsq must be 16-byte aligned", fn);
  if (heads * 2 > 64)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: %d heads give %d partial sums per token, at most 64", fn,
                     heads, heads * 2);
  PrepArgs aq{}, ak{};
  int rc;
  // q: statistics only, no x read (any valid tensor satisfies the checks)
  if ((rc = rms_prep_args(fn, k, nullptr, batch, seqlen, heads, head_dim, nullptr, eps, nullptr,
                          nullptr, inv_rms_q, &aq)))
    return rc;
  if ((rc = rms_prep_args(fn, k, k_out, batch, seqlen, heads, head_dim, gamma_k, eps, rope_cos,
                          rope_sin, nullptr, &ak)))
    return rc;
  if ((int64_t)batch * seqlen * heads == 0) return WAN_OK;
  aq.sumsq = ak.sumsq = sumsq;
  aq.sumsq_parts = ak.sumsq_parts = heads * 2;
  aq.sumsq_first = 0;
  ak.sumsq_first = heads * 2;
  return launch_rms_prep2(aq, ak, static_cast<hipStream_t>(stream));
}

int wan_flash_attn_qnorm(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out, int batch,
                         int heads, int seqlen_q, int seqlen_k, int head_dim,
                         const float* inv_rms_q, const void* gamma_q, const float* rope_cos,
                         const float* rope_sin, float softmax_scale, const int32_t* seqlen_k_dev,
                         void* stream) {
  const char* fn = "wan_flash_attn_qnorm";
  int rc;
  if ((rc = check_scale(fn, softmax_scale))) return rc;
  if ((rc = check_dims(fn, batch, heads, seqlen_q, seqlen_k, head_dim))) return rc;
  if ((rc = check_tensor(fn, "q", q, batch, seqlen_q, heads))) return rc;
  if ((rc = check_tensor(fn, "k", k, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "v", v, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "out", out, batch, seqlen_q, heads))) return rc;
  if (batch == 0 || heads == 0 || seqlen_q == 0) return WAN_OK;
  if (!inv_rms_q || !gamma_q || !aligned16(gamma_q))
    return set_error(WAN_ERR_INVALID, "%s: inv_rms_q and a 16-byte aligned gamma_q are required", fn);
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: rope_cos and rope_sin must both be given or both NULL", fn);
  if (rope_cos && (!aligned16(rope_cos) || !aligned16(rope_sin)))
    return set_error(WAN_ERR_INVALID, "%s: rope tables must be 16-byte aligned", fn);
  FlashArgs a{};
  a.q = as_t4(q);
  a.k = as_t4(k);
  a.v = as_t4(v);
  a.o = static_cast<bf16*>(out.data);
  a.o_sb = out.batch_stride;
  a.o_st = out.token_stride;
  a.o_sh = out.head_stride;
  a.B = batch;
  a.H = heads;
  a.Lq = seqlen_q;
  a.Lk = seqlen_k;
  a.seqlen_k = seqlen_k_dev;
  a.seqlen_all = seqlen_k;
  a.scale = softmax_scale;
  a.qprep = rope_cos ? kQNormRope : kQNorm;
  a.inv_rms_q = inv_rms_q;
  a.gamma_q = static_cast<const bf16*>(gamma_q);
  a.cos = rope_cos;
  a.sin = rope_sin;
  return launch_flash_fwd(a, static_cast<hipStream_t>(stream));
}

int wan_self_attn_fused(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out, int batch,
                        int heads, int seqlen, int head_dim, const void* gamma_q,
                        const void* gamma_k, float eps, const float* rope_cos,
                        const float* rope_sin, float softmax_scale, void* workspace,
                        size_t workspace_bytes, void* stream) {
  const char* fn = "wan_self_attn_fused";
  int rc;
  if ((rc = check_scale(fn, softmax_scale))) return rc;
  if ((rc = check_dims(fn, batch, heads, seqlen, seqlen, head_dim))) return rc;
  if ((rc = check_tensor(fn, "q", q, batch, seqlen, heads))) return rc;
  if ((rc = check_tensor(fn, "k", k, batch, seqlen, heads))) return rc;
  if ((rc = check_tensor(fn, "v", v, batch, seqlen, heads))) return rc;
  if ((rc = check_tensor(fn, "out", out, batch, seqlen, heads))) return rc;
  if (batch == 0 || heads == 0 || seqlen == 0) return WAN_OK;
  if (!gamma_q || !gamma_k || !rope_cos || !rope_sin)
    return set_error(WAN_ERR_INVALID, "%s: gamma_q, gamma_k, rope_cos and rope_sin are required", fn);
  if (!aligned16(gamma_q) || !aligned16(gamma_k) || !aligned16(rope_cos) || !aligned16(rope_sin))
    return set_error(WAN_ERR_INVALID, "%s: gamma and rope tables must be 16-byte aligned", fn);
  if (!(eps >= 0.f)) return set_error(WAN_ERR_INVALID, "%s: eps must be >= 0", fn);
  const size_t need = wan_self_attn_fused_workspace(batch, heads, seqlen);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(WAN_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", fn, need,
                     workspace ? workspace_bytes : (size_t)0);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign)
    return set_error(WAN_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  const size_t rows = (size_t)batch * seqlen;
  float* inv_q = static_cast<float*>(workspace);
  void* khat = static_cast<char*>(workspace) + align_up(rows * sizeof(float));
  const wan_tensor kt{khat, (int64_t)seqlen * heads * kHeadDim, (int64_t)heads * kHeadDim, kHeadDim};
  if ((rc = wan_rms_norm_qk(q, k, khat, batch, seqlen, heads, head_dim, gamma_k, eps, rope_cos,
                            rope_sin, inv_q, stream)))
    return rc;
  return wan_flash_attn_qnorm(q, kt, v, out, batch, heads, seqlen, seqlen, head_dim, inv_q, gamma_q,
                              rope_cos, rope_sin, softmax_scale, nullptr, stream);
}

size_t wan_cross_attn_fused_workspace(int batch, int heads, int seqlen_q) {
  (void)heads;
  if (batch <= 0 || seqlen_q <= 0) return 0;
  return align_up((size_t)batch * seqlen_q * sizeof(float));
}

}  // extern "C"

namespace wan {
// Library-owned scratch of wan_cross_attn_fused_noalloc: the fp32 inverse RMS of each
// query row, WAN_NOALLOC_MAX_ROWS rows (512 KB) per GPU, held until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: its device
// address is looked up once per device with hipGetSymbolAddress (that device current)
// and only that address is handed to the kernels.
__device__ __align__(256) float scratch[WAN_NOALLOC_MAX_ROWS];
}  // namespace wan

namespace {

// Validation shared by the two fused cross-attention entry points (everything but the
// workspace).  Returns WAN_OK, or an error code with the message set.
int check_cross_fused(const char* fn, const wan_tensor& q, const wan_tensor& k, const wan_tensor& v,
                      const wan_tensor& out, int batch, int heads, int seqlen_q, int seqlen_k,
                      int head_dim, const void* gamma_q, float eps, float softmax_scale) {
  int rc;
  if ((rc = check_scale(fn, softmax_scale))) return rc;
  if ((rc = check_dims(fn, batch, heads, seqlen_q, seqlen_k, head_dim))) return rc;
  if ((rc = check_tensor(fn, "q", q, batch, seqlen_q, heads))) return rc;
  if ((rc = check_tensor(fn, "k", k, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "v", v, batch, seqlen_k, heads))) return rc;
  if ((rc = check_tensor(fn, "out", out, batch, seqlen_q, heads))) return rc;
  if (batch == 0 || heads == 0 || seqlen_q == 0) return WAN_OK;
  if (!gamma_q || !aligned16(gamma_q))
    return set_error(WAN_ERR_INVALID, "%s: gamma_q must be a 16-byte aligned pointer", fn);
  if (!(eps >= 0.f)) return set_error(WAN_ERR_INVALID, "%s: eps must be >= 0", fn);
  return WAN_OK;
}

// The two launches of a fused cross-attention, with the per-row inverse RMS of q in inv_q.
int cross_fused_launch(const wan_tensor& q, const wan_tensor& k, const wan_tensor& v,
                       const wan_tensor& out, int batch, int heads, int seqlen_q, int seqlen_k,
                       int head_dim, const void* gamma_q, float eps, float softmax_scale,
                       const int32_t* seqlen_k_dev, float* inv_q, void* stream) {
  int rc;
  if ((rc = wan_rms_norm(q, nullptr, batch, seqlen_q, heads, head_dim, nullptr, eps, nullptr,
                         nullptr, inv_q, stream)))
    return rc;
  return wan_flash_attn_qnorm(q, k, v, out, batch, heads, seqlen_q, seqlen_k, head_dim, inv_q,
                              gamma_q, nullptr, nullptr, softmax_scale, seqlen_k_dev, stream);
}

constexpr int kMaxDevices = 64;
float* g_scratch_dev[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The current device's copy of `scratch`, looked up by wan_attn_init() or on the first
// no-allocation call on that device.
int device_scratch(const char* fn, float** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(WAN_ERR_LAUNCH, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: device %d beyond the %d devices supported", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(WAN_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                       hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_dev[dev];
  return WAN_OK;
}

}  // namespace

extern "C" {

int wan_attn_init(void) {
  float* p = nullptr;
  (void)device_cu_count();
  return device_scratch("wan_attn_init", &p);
}

int wan_cross_attn_fused(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out, int batch,
                         int heads, int seqlen_q, int seqlen_k, int head_dim, const void* gamma_q,
                         float eps, float softmax_scale, const int32_t* seqlen_k_dev,
                         void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "wan_cross_attn_fused";
  int rc;
  if ((rc = check_cross_fused(fn, q, k, v, out, batch, heads, seqlen_q, seqlen_k, head_dim,
                              gamma_q, eps, softmax_scale)))
    return rc;
  if (batch == 0 || heads == 0 || seqlen_q == 0) return WAN_OK;
  const size_t need = wan_cross_attn_fused_workspace(batch, heads, seqlen_q);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(WAN_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", fn, need,
                     workspace ? workspace_bytes : (size_t)0);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign)
    return set_error(WAN_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  return cross_fused_launch(q, k, v, out, batch, heads, seqlen_q, seqlen_k, head_dim, gamma_q, eps,
                            softmax_scale, seqlen_k_dev, static_cast<float*>(workspace), stream);
}

int wan_cross_attn_fused_noalloc(wan_tensor q, wan_tensor k, wan_tensor v, wan_tensor out,
                                 int batch, int heads, int seqlen_q, int seqlen_k, int head_dim,
                                 const void* gamma_q, float eps, float softmax_scale,
                                 const int32_t* seqlen_k_dev, void* stream) {
  const char* fn = "wan_cross_attn_fused_noalloc";
  int rc;
  if ((rc = check_cross_fused(fn, q, k, v, out, batch, heads, seqlen_q, seqlen_k, head_dim,
                              gamma_q, eps, softmax_scale)))
    return rc;
  if ((int64_t)batch * seqlen_q > (int64_t)WAN_NOALLOC_MAX_ROWS)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: batch*seqlen_q=%lld exceeds the static scratch of %d rows",
                     fn, (long long)batch * seqlen_q, WAN_NOALLOC_MAX_ROWS);
  if (batch == 0 || heads == 0 || seqlen_q == 0) return WAN_OK;
  float* inv_q = nullptr;
  if ((rc = device_scratch(fn, &inv_q))) return rc;
  return cross_fused_launch(q, k, v, out, batch, heads, seqlen_q, seqlen_k, head_dim, gamma_q, eps,
                            softmax_scale, seqlen_k_dev, inv_q, stream);
}

int wan_rope(wan_tensor x, void* out, int batch, int seqlen, int heads, int head_dim,
             const float* rope_cos, const float* rope_sin, void* stream) {
  const char* fn = "wan_rope";
  int rc;
  if ((rc = check_dims(fn, batch, heads, seqlen, seqlen, head_dim))) return rc;
  if ((rc = check_tensor(fn, "x", x, batch, seqlen, heads))) return rc;
  if ((int64_t)batch * seqlen * heads == 0) return WAN_OK;
  if (!out || !aligned16(out)) return set_error(WAN_ERR_INVALID, "%s: out must be a 16-byte aligned pointer", fn);
  if (!rope_cos || !rope_sin || !aligned16(rope_cos) || !aligned16(rope_sin))
    return set_error(WAN_ERR_INVALID, "%s: rope tables must be 16-byte aligned pointers", fn);
  RopeArgs a{};
  a.x = as_t4(x);
  a.B = batch;
  a.L = seqlen;
  a.H = heads;
  a.cos = rope_cos;
  a.sin = rope_sin;
  a.out = static_cast<bf16*>(out);
  return launch_rope(a, static_cast<hipStream_t>(stream));
}

int wan_qkv_proj_sumsq(const void* x, const void* w, const void* bias, void* out, float* sumsq,
                       int M, int N, int K, int64_t ldx, int64_t ldw, int64_t ldo, int sq_cols,
                       void* stream) {
  const char* fn = "wan_qkv_proj_sumsq";
  if (M < 0 || N <= 0 || K <= 0)
    return set_error(WAN_ERR_INVALID, "%s: bad sizes (M=%d N=%d K=%d)", fn, M, N, K);
  if (N % 256 != 0 || K % 64 != 0)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: N=%d must be a multiple of 256 and K=%d of 64", fn, N, K);
  if (sq_cols < 0 || sq_cols % 64 != 0 || sq_cols > N)
    return set_error(WAN_ERR_INVALID, "%s: sq_cols=%d must be a multiple of 64 in [0, N]", fn, sq_cols);
  if (ldx < K || ldw < K || ldo < N || ldx % 8 || ldw % 8 || ldo % 8)
    return set_error(WAN_ERR_INVALID, "%s: row strides (%lld, %lld, %lld) must cover the rows and be "
                     "multiples of 8 elements", fn, (long long)ldx, (long long)ldw, (long long)ldo);
  // a tile's 256 rows are addressed with 32-bit byte offsets
  if (ldx >= (int64_t(1) << 23) || ldw >= (int64_t(1) << 23))
    return set_error(WAN_ERR_UNSUPPORTED, "%s: row strides must be below 2^23 elements", fn);
  // x, w, bias and out are always read or written when M > 0; sumsq only when sq_cols > 0
  if (M > 0 && (x == nullptr || w == nullptr || bias == nullptr || out == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: x, w, bias and out must not be NULL", fn);
  if (M > 0 && sq_cols > 0 && sumsq == nullptr)
    return set_error(WAN_ERR_INVALID, "%s: sumsq must not be NULL when sq_cols > 0", fn);
  const void* ptrs[] = {x, w, bias, out, sumsq};
  for (const void* p : ptrs)
    if (!aligned16(p))
      return set_error(WAN_ERR_INVALID, "%s: operands must be 16-byte aligned device pointers", fn);
  GemmArgs a;
  a.x = static_cast<const bf16*>(x);
  a.w = static_cast<const bf16*>(w);
  a.bias = static_cast<const bf16*>(bias);
  a.out = static_cast<bf16*>(out);
  a.sumsq = sumsq;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ldx = ldx;
  a.ldw = ldw;
  a.ldo = ldo;
  a.sq_cols = sq_cols;
  return launch_gemm_rowsq(a, static_cast<hipStream_t>(stream));
}

int wan_adaln_ex(const void* x, const void* y, void* x_out, void* h_out, int batch, int seqlen,
                 int dim, const void* e, int frames, int gate_idx, const void* e_mod, int mod_rows,
                 int shift_idx, int scale_idx, const void* ln_weight, const void* ln_bias, float eps,
                 void* stream) {
  const char* fn = e_mod ? "wan_adaln_ex" : "wan_adaln";
  if (batch < 0 || seqlen < 0 || dim <= 0 || frames <= 0)
    return set_error(WAN_ERR_INVALID, "%s: bad sizes (batch=%d seqlen=%d dim=%d frames=%d)", fn,
                     batch, seqlen, dim, frames);
  if (dim % 8 != 0 || dim > 8192)
    return set_error(WAN_ERR_UNSUPPORTED, "%s: dim=%d must be a multiple of 8 and <= 8192", fn, dim);
  if (seqlen % frames != 0)
    return set_error(WAN_ERR_INVALID, "%s: seqlen=%d is not a multiple of frames=%d", fn, seqlen,
                     frames);
  if (e_mod == nullptr) {
    e_mod = e;
    mod_rows = 6;
  } else if (mod_rows < 1 || mod_rows > 6) {
    return set_error(WAN_ERR_INVALID, "%s: mod_rows=%d must be in [1, 6]", fn, mod_rows);
  }
  if (gate_idx < -1 || gate_idx > 5 || shift_idx < -1 || shift_idx >= mod_rows || scale_idx < -1 ||
      scale_idx >= mod_rows || ((shift_idx < 0) != (scale_idx < 0)))
    return set_error(WAN_ERR_INVALID, "%s: modulation rows gate=%d shift=%d scale=%d out of range",
                     fn, gate_idx, shift_idx, scale_idx);
  if (x == nullptr || (y == nullptr && x_out != nullptr) || (gate_idx >= 0 && y == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: x is NULL, or x_out / a gate given without y", fn);
  if (h_out == nullptr && (shift_idx >= 0 || ln_weight != nullptr))
    return set_error(WAN_ERR_INVALID, "%s: modulation or LayerNorm weights given without h_out", fn);
  if ((gate_idx >= 0 && e == nullptr) || (shift_idx >= 0 && e_mod == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: modulation rows requested but e is NULL", fn);
  if ((ln_weight == nullptr) != (ln_bias == nullptr))
    return set_error(WAN_ERR_INVALID, "%s: LayerNorm weight and bias must be given together", fn);
  const void* ptrs[] = {x, y, x_out, h_out, e, e_mod, ln_weight, ln_bias};
  for (const void* p : ptrs)
    if (!aligned16(p)) return set_error(WAN_ERR_INVALID, "%s: operands must be 16-byte aligned", fn);
  AdaLNArgs a;
  a.x = static_cast<const bf16*>(x);
  a.y = static_cast<const bf16*>(y);
  a.x_out = static_cast<bf16*>(x_out);
  a.h_out = static_cast<bf16*>(h_out);
  a.B = batch;
  a.L = seqlen;
  a.C = dim;
  a.F = frames;
  a.e = static_cast<const bf16*>(e);
  a.gate_idx = gate_idx;
  a.e_mod = static_cast<const bf16*>(e_mod);
  a.mod_rows = mod_rows;
  a.shift_idx = shift_idx;
  a.scale_idx = scale_idx;
  a.ln_w = static_cast<const bf16*>(ln_weight);
  a.ln_b = static_cast<const bf16*>(ln_bias);
  a.eps = eps;
  return launch_adaln(a, static_cast<hipStream_t>(stream));
}

int wan_adaln(const void* x, const void* y, void* x_out, void* h_out, int batch, int seqlen,
              int dim, const void* e, int frames, int gate_idx, int shift_idx, int scale_idx,
              const void* ln_weight, const void* ln_bias, float eps, void* stream) {
  return wan_adaln_ex(x, y, x_out, h_out, batch, seqlen, dim, e, frames, gate_idx, nullptr, 6,
                      shift_idx, scale_idx, ln_weight, ln_bias, eps, stream);
}

}  // extern "C"
