// api.cpp -- the entry points of include/e5m2effma.h and include/e5m2effma_ext.h.
//
// Each entry point opens a Call (which empties the calling thread's message), states its argument
// rules in order -- the first broken rule decides the status and the message -- then resolves the
// current device and hands plain values to a kernel launcher.  The rules, their order and their
// message texts are the reference's contract (src/gemm_e5m2effma.cu:55-81, src/e5m2effma.cu:88-95,
// src/adamw_e5m2effma.cu:131-147): callers and tests match on them.  No rule touches the device.
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "e5m2effma_ext.h"
#include "e5ma_host.hpp"
#include "e5ma_tuned.h"

namespace e5ma {

// ---- the thread's message -------------------------------------------------------------------------
namespace {
constexpr size_t kMessageBytes = 1024;
thread_local char t_message[kMessageBytes];
}  // namespace

const char *thread_message() { return t_message; }

Call::Call() { t_message[0] = 0; }

Call &Call::need(bool holds, e5ma_status s, const char *fmt, ...) {
  if (holds || status_ != E5MA_OK) return *this;
  status_ = s;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_message, kMessageBytes, fmt, ap);
  va_end(ap);
  return *this;
}

e5ma_status Call::hip(hipError_t e, const char *what) {
  need(e == hipSuccess, E5MA_HIP_ERROR, "%s: HIP error %d (%s): %s", what, (int)e, hipGetErrorName(e),
       hipGetErrorString(e));
  return status_;
}

// ---- devices --------------------------------------------------------------------------------------
namespace {

// tuned launch choices per (architecture, CU count), written by the tuner (e5m2effma_amd/tune/tune.cpp)
struct TunedEntry {
  const char *arch;
  int cus;
  Tuning t;
};
const TunedEntry kTuned[] = {E5MA_TUNED_ENTRIES{nullptr, 0, {}}};

Tuning tuned_for(const char *arch, int cus) {
  for (const TunedEntry *e = kTuned; e->arch; ++e) {
    const size_t len = strlen(e->arch);
    const bool same_arch = strncmp(arch, e->arch, len) == 0 && (arch[len] == 0 || arch[len] == ':');
    if (same_arch && e->cus == cus) return e->t;
  }
  return Tuning{};
}

// filled once per device, race-free (the reference's per-device cache, src/e5m2effma.cu:31-51, is lazy
// and unsynchronised)
struct DeviceSlot {
  std::once_flag once;
  DeviceInfo info;
};
DeviceSlot g_devices[kMaxDevices];

}  // namespace

const DeviceInfo &device_info(int dev) {
  DeviceSlot &slot = g_devices[dev];
  std::call_once(slot.once, [&slot, dev] {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    DeviceInfo &d = slot.info;
    d.cus = p.multiProcessorCount;
    snprintf(d.arch, sizeof d.arch, "%s", p.gcnArchName);
    d.supported = strncmp(p.gcnArchName, "gfx950", 6) == 0;
    d.tune = tuned_for(p.gcnArchName, d.cus);
  });
  return slot.info;
}

e5ma_status resolve_device(Call &call, int *dev_out) {
  int dev = -1;
  if (call.hip(hipGetDevice(&dev), "hipGetDevice")) return call.status();
  call.need(dev >= 0 && dev < kMaxDevices, E5MA_NOT_SUPPORTED, "device %d: the library handles device indices below %d",
            dev, kMaxDevices);
  if (!call.ok()) return call.status();
  const DeviceInfo &d = device_info(dev);
  call.need(d.supported, E5MA_NOT_SUPPORTED,
            "device %d is %s, but this build of the library has code for gfx950 (MI355X) only", dev,
            d.arch[0] ? d.arch : "unknown");
  *dev_out = dev;
  return call.status();
}

namespace {

bool known_dtype(int t) { return t >= E5MA_E4M3 && t <= E5MA_E5M2; }
bool gemm_operand(int t) { return is_fp8(t) || t == E5MA_BF16 || t == E5MA_FP32; }
bool known_op(int o) { return o == E5MA_OP_N || o == E5MA_OP_T; }
bool has_data(const e5ma_tensor *t) { return t && t->data; }
bool has_data_pair(const e5ma_tensor *x, const e5ma_tensor *y) { return has_data(x) && has_data(y); }
bool aligned(const void *p, uintptr_t bytes) { return ((uintptr_t)p & (bytes - 1)) == 0; }
// a descriptor's field, or a stand-in when the descriptor is absent (rules evaluate their arguments)
int dtype_of(const e5ma_tensor *t) { return t ? (int)t->dtype : -1; }
int scaling_of(const e5ma_tensor *t) { return t ? (int)t->scaling : (int)E5MA_SCALING_TENSOR; }

// The epilogue of one GEMM call (include/e5m2effma.h).  Scale pointers are taken only for FP8
// tensors; with beta != 0 the epilogue reads C, or D itself when C is NULL (TE's accumulate into D).
dev::Epilogue epilogue_of(float alpha, const e5ma_tensor *A, const e5ma_tensor *B, float beta, const e5ma_tensor *C,
                          int ldc, const e5ma_tensor *D, int ldd, const e5ma_tensor *bias) {
  const auto fp8_scale = [](const e5ma_tensor *t, const float *s) { return is_fp8(t->dtype) ? s : nullptr; };
  const e5ma_tensor *src = beta == 0.f ? nullptr : has_data(C) ? C : D;
  dev::Epilogue e{};
  e.alpha = alpha;
  e.beta = beta;
  e.sa = fp8_scale(A, A->scale_inv);
  e.sb = fp8_scale(B, B->scale_inv);
  e.sa_vec = A->scaling == E5MA_SCALING_OUTER;
  e.sb_vec = B->scaling == E5MA_SCALING_OUTER;
  e.c = src ? src->data : nullptr;
  e.ldc = src == nullptr ? 0 : src == D ? ldd : ldc;
  e.c_dtype = src ? (int)src->dtype : (int)E5MA_FP32;
  e.c_sinv = src ? fp8_scale(src, src->scale_inv) : nullptr;
  e.d = D->data;
  e.ldd = ldd;
  e.d_dtype = D->dtype;
  e.d_scale = fp8_scale(D, D->scale);
  e.amax = D->amax;
  e.bias = has_data(bias) ? bias->data : nullptr;
  e.bias_dtype = bias ? (int)bias->dtype : (int)E5MA_FP32;
  return e;
}

// GEMV routing (the reference's rule, src/gemm_e5m2effma.cu:100-102): n <= 8, A FP8 and both
// operands K-contiguous
bool routes_to_gemv(int n, bool akc, bool bkc, int at) { return n <= 8 && akc && bkc && is_fp8(at); }

}  // namespace

// e5ma_gemm and its variants: the rules of src/gemm_e5m2effma.cu:55-81, in that order, then the launch.
e5ma_status gemm_entry(const char *name, e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                       const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                       const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd, const e5ma_tensor *bias,
                       const WorkspaceSource &src, hipStream_t stream) {
  Call call;
  const bool reads_c = beta != 0.f && has_data(C);
  call.need(has_data(A) && has_data(B) && has_data(D), E5MA_INVALID_VALUE, "%s: A, B, D or their data is NULL", name)
      .need(known_op(transa) && known_op(transb), E5MA_INVALID_VALUE, "%s: transa / transb must be E5MA_OP_N or E5MA_OP_T",
            name)
      .need(m >= 0 && n >= 0 && k >= 0, E5MA_INVALID_VALUE, "%s: negative size (m=%d n=%d k=%d)", name, m, n, k)
      .need(known_dtype(dtype_of(D)), E5MA_INVALID_VALUE, "%s: invalid D dtype %d", name, dtype_of(D))
      .need(gemm_operand(dtype_of(A)) && gemm_operand(dtype_of(B)), E5MA_NOT_SUPPORTED,
            "%s: A and B must be E5M2, E4M3, BF16 or FP32 (got dtypes %d, %d)", name, dtype_of(A), dtype_of(B));
  if (!call.ok() || m == 0 || n == 0) return call.status();  // an empty output is done before any layout rule
  const bool akc = transa == E5MA_OP_T, bkc = transb == E5MA_OP_N;
  const int a_min = akc ? k : m, b_min = bkc ? k : n;
  call.need(k % 16 == 0, E5MA_INVALID_VALUE, "%s: k = %d is not a multiple of 16", name, k)
      .need(lda % 16 == 0 && ldb % 16 == 0, E5MA_INVALID_VALUE, "%s: lda = %d / ldb = %d must be multiples of 16", name,
            lda, ldb)
      .need(aligned(A->data, 16) && aligned(B->data, 16), E5MA_INVALID_VALUE, "%s: A and B must be 16-byte aligned", name)
      .need(lda >= a_min, E5MA_INVALID_VALUE, "%s: lda = %d < %d", name, lda, a_min)
      .need(ldb >= b_min, E5MA_INVALID_VALUE, "%s: ldb = %d < %d", name, ldb, b_min)
      .need(ldd >= m, E5MA_INVALID_VALUE, "%s: ldd = %d < m = %d", name, ldd, m)
      .need(!has_data(bias) || known_dtype(dtype_of(bias)), E5MA_INVALID_VALUE, "%s: invalid bias dtype %d", name,
            dtype_of(bias))
      .need(!reads_c || known_dtype(dtype_of(C)), E5MA_INVALID_VALUE, "%s: invalid C dtype %d", name, dtype_of(C))
      .need(!reads_c || ldc >= m, E5MA_INVALID_VALUE, "%s: ldc = %d < m = %d", name, ldc, m);
  const auto scaling_known = [](const e5ma_tensor *t) {
    return t->scaling == E5MA_SCALING_TENSOR || t->scaling == E5MA_SCALING_OUTER;
  };
  const auto outer_ok = [](const e5ma_tensor *t) {
    return t->scaling != E5MA_SCALING_OUTER || (is_fp8(t->dtype) && t->scale_inv);
  };
  call.need(scaling_known(A) && scaling_known(B), E5MA_INVALID_VALUE, "%s: invalid scaling of A or B", name)
      .need(outer_ok(A) && outer_ok(B), E5MA_INVALID_VALUE,
            "%s: E5MA_SCALING_OUTER needs an FP8 operand with a scale_inv vector", name)
      .need(scaling_of(C) == E5MA_SCALING_TENSOR && scaling_of(D) == E5MA_SCALING_TENSOR &&
                scaling_of(bias) == E5MA_SCALING_TENSOR,
            E5MA_INVALID_VALUE, "%s: C, D and bias take per-tensor scaling only", name);
  int dev = 0;
  if (!call.ok() || resolve_device(call, &dev)) return call.status();
  const DeviceInfo &di = device_info(dev);
  const Workspace ws = src.per_device ? src.per_device(dev, call) : src.given;
  if (src.per_device && call.ok()) {
    const size_t want = routes_to_gemv(n, akc, bkc, A->dtype)
                            ? 0
                            : gemm_workspace_bytes(A->dtype, B->dtype, akc, bkc, m, n, k, lda, ldb, di);
    call.need(want <= ws.bytes, E5MA_INVALID_VALUE,
              "%s: this GEMM's split-K partials need %zu bytes, more than the library's scratch of %zu bytes", name,
              want, ws.bytes);
  }
  if (!call.ok()) return call.status();

  const dev::Epilogue e = epilogue_of(alpha, A, B, beta, C, ldc, D, ldd, bias);
  const uint8_t *a = (const uint8_t *)A->data, *b = (const uint8_t *)B->data;
  const hipError_t err = routes_to_gemv(n, akc, bkc, A->dtype)
                             ? launch_gemv(A->dtype, B->dtype, a, lda, b, ldb, m, n, k, e, di, stream)
                             : launch_gemm(A->dtype, B->dtype, akc, bkc, a, lda, b, ldb, m, n, k, e, di, ws, stream);
  char what[64];
  snprintf(what, sizeof what, "%s: kernel launch", name);
  return call.hip(err, what);
}

}  // namespace e5ma

using e5ma::Call;

extern "C" const char *e5ma_last_error(void) { return e5ma::thread_message(); }

extern "C" const char *e5ma_status_string(e5ma_status s) {
  // value 3 keeps the reference's name (include/e5m2effma.h there)
  static const char *const kNames[] = {"E5MA_OK", "E5MA_INVALID_VALUE", "E5MA_NOT_SUPPORTED", "E5MA_CUDA_ERROR"};
  const int i = (int)s;
  return i >= 0 && i < 4 ? kNames[i] : "unknown e5ma_status";
}

// rules of src/e5m2effma.cu:88-95
extern "C" e5ma_status e5ma_cast(const e5ma_tensor *src, const e5ma_tensor *dst, size_t count, hipStream_t stream) {
  Call call;
  call.need(e5ma::has_data_pair(src, dst), E5MA_INVALID_VALUE, "e5ma_cast: src / dst or their data is NULL");
  if (!call.ok()) return call.status();
  call.need(e5ma::known_dtype(src->dtype) && e5ma::known_dtype(dst->dtype), E5MA_INVALID_VALUE, "e5ma_cast: invalid dtype (src %d, dst %d)",
            (int)src->dtype, (int)dst->dtype)
      .need(src->scaling == E5MA_SCALING_TENSOR && dst->scaling == E5MA_SCALING_TENSOR, E5MA_INVALID_VALUE,
            "e5ma_cast: per-tensor scaling only");
  int dev = 0;
  if (!call.ok() || count == 0 || e5ma::resolve_device(call, &dev)) return call.status();
  const float *sinv = e5ma::is_fp8(src->dtype) ? src->scale_inv : nullptr;
  const float *qscale = e5ma::is_fp8(dst->dtype) ? dst->scale : nullptr;
  return call.hip(e5ma::launch_cast(src->dtype, dst->dtype, src->data, dst->data, count, sinv, qscale, dst->amax,
                                    e5ma::device_info(dev).tune, stream),
                  "e5ma_cast: kernel launch");
}

// No C-ABI counterpart in the reference: its Float8Tensor.from_float runs these steps as torch
// operations plus e5ma_cast (binds/python/e5m2effma/tensor.py:60-74)
extern "C" e5ma_status e5ma_quantize(const e5ma_tensor *src, const e5ma_tensor *dst, size_t rows, size_t cols,
                                     float qmax, float *scale_inv, float *amax_out, hipStream_t stream) {
  Call call;
  call.need(e5ma::has_data_pair(src, dst) && scale_inv, E5MA_INVALID_VALUE,
            "e5ma_quantize: src / dst, their data or scale_inv is NULL");
  if (!call.ok()) return call.status();
  const bool per_row = dst->scaling == E5MA_SCALING_OUTER;
  call.need(e5ma::known_dtype(src->dtype) && e5ma::is_fp8(dst->dtype), E5MA_INVALID_VALUE,
            "e5ma_quantize: src dtype %d / dst dtype %d (dst must be E5MA_E4M3 or E5MA_E5M2)", (int)src->dtype,
            (int)dst->dtype)
      .need(src->scaling == E5MA_SCALING_TENSOR, E5MA_INVALID_VALUE, "e5ma_quantize: src takes per-tensor scaling only")
      .need(per_row || dst->scaling == E5MA_SCALING_TENSOR, E5MA_INVALID_VALUE, "e5ma_quantize: invalid dst scaling %d",
            (int)dst->scaling)
      .need(qmax > 0.f && !isinf(qmax), E5MA_INVALID_VALUE, "e5ma_quantize: qmax = %g must be positive and finite",
            (double)qmax);
  if (!call.ok() || rows == 0 || cols == 0) return call.status();
  // per row, a launch has up to 256 threads per row and HIP's grid holds fewer than 2^32 threads
  call.need(cols <= SIZE_MAX / rows, E5MA_INVALID_VALUE, "e5ma_quantize: rows x cols overflows")
      .need(!per_row || rows < ((size_t)1 << 24), E5MA_INVALID_VALUE,
            "e5ma_quantize: per-row scaling takes at most %d rows, got %zu", (1 << 24) - 1, rows);
  int dev = 0;
  if (!call.ok() || e5ma::resolve_device(call, &dev)) return call.status();
  const float *sinv = e5ma::is_fp8(src->dtype) ? src->scale_inv : nullptr;
  return call.hip(e5ma::launch_quantize(src->dtype, dst->dtype, src->data, dst->data, rows, cols, sinv, qmax, per_row,
                                        scale_inv, amax_out, e5ma::device_info(dev).tune, stream),
                  "e5ma_quantize: kernel launch");
}

namespace {

// The coefficients of one step, formed in double and rounded to FP32 once (reference
// src/adamw_e5m2effma.cu:150-157)
e5ma::AdamCoefficients adam_coefficients(const e5ma_adam_config &c) {
  const auto correction = [&c](float beta) {
    return c.bias_correction ? (float)(1.0 / (1.0 - pow((double)beta, c.step))) : 1.f;
  };
  e5ma::AdamCoefficients a;
  a.grad_mul = c.grad_scale == 0.f ? 1.f : c.grad_scale;
  a.l2 = c.weight_decay;
  a.b1 = c.beta1;
  a.c1 = (float)(1.0 - (double)c.beta1);
  a.b2 = c.beta2;
  a.c2 = (float)(1.0 - (double)c.beta2);
  a.corr1 = correction(c.beta1);
  a.corr2 = correction(c.beta2);
  a.eps = c.eps;
  a.decay = (float)((double)c.lr * c.weight_decay);
  a.lr = c.lr;
  a.decoupled = c.adamw ? 1 : 0;
  return a;
}

}  // namespace

// rules of src/adamw_e5m2effma.cu:131-147
extern "C" e5ma_status e5ma_adam(const e5ma_adam_config *cfg, size_t count, const e5ma_tensor *param,
                                 const e5ma_tensor *grad, const e5ma_tensor *exp_avg,
                                 const e5ma_tensor *exp_avg_sq, const e5ma_tensor *param_fp8,
                                 hipStream_t stream) {
  Call call;
  const auto state = [](int t) { return t == E5MA_FP32 || t == E5MA_BF16; };
  call.need(cfg && e5ma::has_data_pair(param, grad) && e5ma::has_data_pair(exp_avg, exp_avg_sq), E5MA_INVALID_VALUE,
            "e5ma_adam: cfg, param, grad, exp_avg, exp_avg_sq or their data is NULL");
  if (!call.ok()) return call.status();
  const bool copy = param_fp8 && param_fp8->data;
  call.need(cfg->step >= 1, E5MA_INVALID_VALUE, "e5ma_adam: step = %d, must be >= 1", cfg->step)
      .need(state(param->dtype), E5MA_NOT_SUPPORTED, "e5ma_adam: param must be FP32 or BF16 (dtype %d)", (int)param->dtype)
      .need(state(exp_avg->dtype) && exp_avg_sq->dtype == exp_avg->dtype, E5MA_NOT_SUPPORTED,
            "e5ma_adam: exp_avg and exp_avg_sq must both be FP32 or both BF16 (dtypes %d, %d)", (int)exp_avg->dtype,
            (int)exp_avg_sq->dtype)
      .need(grad->dtype == E5MA_BF16 || grad->dtype == E5MA_FP16 || grad->dtype == E5MA_FP32, E5MA_NOT_SUPPORTED,
            "e5ma_adam: grad must be FP32, BF16 or FP16 (dtype %d)", (int)grad->dtype)
      .need(!copy || e5ma::is_fp8(param_fp8->dtype), E5MA_INVALID_VALUE,
            "e5ma_adam: param_fp8 must have dtype E5MA_E4M3 or E5MA_E5M2 (dtype %d)", copy ? (int)param_fp8->dtype : 0)
      .need(!copy || param_fp8->scaling == E5MA_SCALING_TENSOR, E5MA_INVALID_VALUE,
            "e5ma_adam: param_fp8 takes per-tensor scaling only");
  int dev = 0;
  if (!call.ok() || count == 0 || e5ma::resolve_device(call, &dev)) return call.status();
  uint8_t *q = copy ? (uint8_t *)param_fp8->data : nullptr;
  return call.hip(e5ma::launch_adam(adam_coefficients(*cfg), count, param->dtype, param->data, grad->dtype, grad->data,
                                    exp_avg->dtype, exp_avg->data, exp_avg_sq->data,
                                    copy ? (int)param_fp8->dtype : (int)E5MA_E4M3, q, copy ? param_fp8->scale : nullptr,
                                    copy ? param_fp8->amax : nullptr, e5ma::device_info(dev).tune, stream),
                  "e5ma_adam: kernel launch");
}

// reference src/gemm_e5m2effma.cu:44-104: never splits K, so it needs and allocates no device memory
extern "C" e5ma_status e5ma_gemm(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                                 const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                                 const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                                 const e5ma_tensor *bias, hipStream_t stream) {
  return e5ma::gemm_entry("e5ma_gemm", transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, D, ldd, bias,
                          e5ma::WorkspaceSource{}, stream);
}

// e5ma_gemm with a caller-owned split-K workspace (include/e5m2effma_ext.h)
extern "C" e5ma_status e5ma_gemm_ex(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                                    const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                                    const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                                    const e5ma_tensor *bias, void *workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  {
    Call call;
    call.need(workspace_bytes == 0 || (workspace && e5ma::aligned(workspace, 256)), E5MA_INVALID_VALUE,
              "e5ma_gemm_ex: a workspace of %zu bytes needs a 256-byte aligned pointer", workspace_bytes);
    if (!call.ok()) return call.status();
  }
  e5ma::WorkspaceSource src;
  src.given = e5ma::Workspace{workspace_bytes ? workspace : nullptr, workspace_bytes};
  return e5ma::gemm_entry("e5ma_gemm_ex", transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, D, ldd, bias,
                          src, stream);
}

extern "C" e5ma_status e5ma_gemm_workspace_size(e5ma_op transa, e5ma_op transb, int m, int n, int k,
                                                e5ma_dtype a_dtype, int lda, e5ma_dtype b_dtype, int ldb,
                                                size_t *bytes) {
  Call call;
  call.need(bytes != nullptr, E5MA_INVALID_VALUE, "e5ma_gemm_workspace_size: bytes is NULL")
      .need(e5ma::known_op(transa) && e5ma::known_op(transb), E5MA_INVALID_VALUE,
            "e5ma_gemm_workspace_size: transa / transb must be E5MA_OP_N or E5MA_OP_T")
      .need(m >= 0 && n >= 0 && k >= 0, E5MA_INVALID_VALUE, "e5ma_gemm_workspace_size: negative size (m=%d n=%d k=%d)",
            m, n, k)
      .need(e5ma::gemm_operand(a_dtype) && e5ma::gemm_operand(b_dtype), E5MA_NOT_SUPPORTED,
            "e5ma_gemm_workspace_size: A and B must be E5M2, E4M3, BF16 or FP32 (got dtypes %d, %d)", (int)a_dtype,
            (int)b_dtype);
  if (!call.ok()) return call.status();
  *bytes = 0;
  const bool akc = transa == E5MA_OP_T, bkc = transb == E5MA_OP_N;
  if (m == 0 || n == 0 || k == 0 || k % 16 || e5ma::routes_to_gemv(n, akc, bkc, a_dtype)) return E5MA_OK;
  int dev = 0;
  if (e5ma::resolve_device(call, &dev)) return call.status();
  *bytes = e5ma::gemm_workspace_bytes(a_dtype, b_dtype, akc, bkc, m, n, k, lda, ldb, e5ma::device_info(dev));
  return E5MA_OK;
}
