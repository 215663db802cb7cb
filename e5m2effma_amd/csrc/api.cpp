// api.cpp -- the C ABI (include/e5m2effma.h): argument validation, error state, device check and
// routing to the gfx950 kernels.  Validation order and message texts follow the reference host code
// (src/gemm_e5m2effma.cu:44-104, src/e5m2effma.cu:85-111, src/adamw_e5m2effma.cu:125-168), so callers
// see the same status for the same mistake.  All validation precedes any device call.
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "e5m2effma_ext.h"
#include "e5ma_host.hpp"
#include "e5ma_tuned.h"

namespace e5ma {

static thread_local char g_error[512];

void clear_error() { g_error[0] = 0; }

e5ma_status fail(e5ma_status s, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return s;
}

e5ma_status hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return E5MA_OK;
  return fail(E5MA_HIP_ERROR, "%s: HIP error %d (%s): %s", what, (int)e, hipGetErrorName(e), hipGetErrorString(e));
}

// Tuned launch choices per (architecture, CU count), written by the tuner (e5m2effma_amd/tune/tune.cpp)
struct TunedEntry {
  const char *arch;
  int cus;
  Tuning t;
};
static const TunedEntry kTuned[] = {E5MA_TUNED_ENTRIES{nullptr, 0, {}}};

static Tuning tuning_for(const char *arch, int cus) {
  for (const TunedEntry *e = kTuned; e->arch; ++e) {
    const size_t n = strlen(e->arch);
    if (e->cus == cus && strncmp(arch, e->arch, n) == 0 && (arch[n] == 0 || arch[n] == ':')) return e->t;
  }
  return Tuning{};
}

// Per-device properties, filled once per device (reference src/e5m2effma.cu:31-51 keeps a lazy
// per-device cache; here std::call_once makes the first use race-free).
static constexpr int kMaxDevices = 64;
static DeviceInfo g_dev[kMaxDevices];
static std::once_flag g_dev_once[kMaxDevices];

const DeviceInfo &device_info(int dev) {
  DeviceInfo &d = g_dev[dev & (kMaxDevices - 1)];
  std::call_once(g_dev_once[dev & (kMaxDevices - 1)], [&d, dev] {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    d.cus = p.multiProcessorCount;
    snprintf(d.arch, sizeof d.arch, "%s", p.gcnArchName);
    d.supported = strncmp(p.gcnArchName, "gfx950", 6) == 0;
    d.tune = tuning_for(p.gcnArchName, d.cus);
    d.xcds = 8;
    if (d.supported) {
      hipMemPoolProps props{};
      props.allocType = hipMemAllocationTypePinned;
      props.location.type = hipMemLocationTypeDevice;
      props.location.id = dev;
      hipMemPool_t pool = nullptr;
      if (hipMemPoolCreate(&pool, &props) == hipSuccess) {
        uint64_t keep = UINT64_MAX;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        d.pool = pool;
      } else {
        (void)hipGetLastError();
      }
    }
  });
  return d;
}

e5ma_status check_device(int *dev_out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev_out) *dev_out = dev;
  const DeviceInfo &d = device_info(dev);
  if (d.supported) return E5MA_OK;
  return fail(E5MA_NOT_SUPPORTED, "device %d is %s, but this build of the library has code for gfx950 (MI355X) only",
              dev, d.arch[0] ? d.arch : "unknown");
}

}  // namespace e5ma

using e5ma::fail;
using e5ma::is_fp8;

static bool valid_dtype(int t) { return t >= E5MA_E4M3 && t <= E5MA_E5M2; }

extern "C" const char *e5ma_last_error(void) { return e5ma::g_error; }

extern "C" const char *e5ma_status_string(e5ma_status s) {
  switch ((int)s) {
    case E5MA_OK: return "E5MA_OK";
    case E5MA_INVALID_VALUE: return "E5MA_INVALID_VALUE";
    case E5MA_NOT_SUPPORTED: return "E5MA_NOT_SUPPORTED";
    case E5MA_HIP_ERROR: return "E5MA_CUDA_ERROR";
  }
  return "unknown e5ma_status";
}

// reference src/e5m2effma.cu:85-101
extern "C" e5ma_status e5ma_cast(const e5ma_tensor *src, const e5ma_tensor *dst, size_t count, hipStream_t stream) {
  e5ma::clear_error();
  if (!src || !dst || !src->data || !dst->data) return fail(E5MA_INVALID_VALUE, "e5ma_cast: src / dst or their data is NULL");
  if (!valid_dtype(src->dtype) || !valid_dtype(dst->dtype))
    return fail(E5MA_INVALID_VALUE, "e5ma_cast: invalid dtype (src %d, dst %d)", (int)src->dtype, (int)dst->dtype);
  if (src->scaling != E5MA_SCALING_TENSOR || dst->scaling != E5MA_SCALING_TENSOR)
    return fail(E5MA_INVALID_VALUE, "e5ma_cast: per-tensor scaling only");
  if (count == 0) return E5MA_OK;
  int dev = 0;
  if (e5ma_status st = e5ma::check_device(&dev)) return st;
  const hipError_t err = e5ma::launch_cast(src->dtype, dst->dtype, src->data, dst->data, count,
                                          is_fp8(src->dtype) ? src->scale_inv : nullptr,
                                          is_fp8(dst->dtype) ? dst->scale : nullptr, dst->amax,
                                          e5ma::device_info(dev).tune, stream);
  return e5ma::hip_status(err, "e5ma_cast: kernel launch");
}

// No C-ABI counterpart in the reference: its Float8Tensor.from_float runs these steps as torch
// operations plus e5ma_cast (binds/python/e5m2effma/tensor.py:60-74)
extern "C" e5ma_status e5ma_quantize(const e5ma_tensor *src, const e5ma_tensor *dst, size_t rows, size_t cols,
                                     float qmax, float *scale_inv, float *amax_out, hipStream_t stream) {
  e5ma::clear_error();
  if (!src || !dst || !src->data || !dst->data || !scale_inv)
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: src / dst, their data or scale_inv is NULL");
  if (!valid_dtype(src->dtype) || !is_fp8(dst->dtype))
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: src dtype %d / dst dtype %d (dst must be E5MA_E4M3 or E5MA_E5M2)",
                (int)src->dtype, (int)dst->dtype);
  if (src->scaling != E5MA_SCALING_TENSOR)
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: src takes per-tensor scaling only");
  if (dst->scaling != E5MA_SCALING_TENSOR && dst->scaling != E5MA_SCALING_OUTER)
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: invalid dst scaling %d", (int)dst->scaling);
  if (!(qmax > 0.f) || isinf(qmax))
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: qmax = %g must be positive and finite", (double)qmax);
  if (rows == 0 || cols == 0) return E5MA_OK;
  if (cols > SIZE_MAX / rows) return fail(E5MA_INVALID_VALUE, "e5ma_quantize: rows x cols overflows");
  // per row, a launch has up to 256 threads per row and HIP's grid holds fewer than 2^32 threads
  if (dst->scaling == E5MA_SCALING_OUTER && rows >= ((size_t)1 << 24))
    return fail(E5MA_INVALID_VALUE, "e5ma_quantize: per-row scaling takes at most %d rows, got %zu", (1 << 24) - 1, rows);
  int dev = 0;
  if (e5ma_status st = e5ma::check_device(&dev)) return st;
  const hipError_t err = e5ma::launch_quantize(src->dtype, dst->dtype, src->data, dst->data, rows, cols,
                                               is_fp8(src->dtype) ? src->scale_inv : nullptr, qmax,
                                               dst->scaling == E5MA_SCALING_OUTER, scale_inv, amax_out,
                                               e5ma::device_info(dev).tune, stream);
  return e5ma::hip_status(err, "e5ma_quantize: kernel launch");
}

// reference src/adamw_e5m2effma.cu:125-168
extern "C" e5ma_status e5ma_adam(const e5ma_adam_config *cfg, size_t count, const e5ma_tensor *param,
                                 const e5ma_tensor *grad, const e5ma_tensor *exp_avg,
                                 const e5ma_tensor *exp_avg_sq, const e5ma_tensor *param_fp8,
                                 hipStream_t stream) {
  e5ma::clear_error();
  if (!cfg || !param || !grad || !exp_avg || !exp_avg_sq || !param->data || !grad->data || !exp_avg->data ||
      !exp_avg_sq->data)
    return fail(E5MA_INVALID_VALUE, "e5ma_adam: cfg, param, grad, exp_avg, exp_avg_sq or their data is NULL");
  if (cfg->step < 1) return fail(E5MA_INVALID_VALUE, "e5ma_adam: step = %d, must be >= 1", cfg->step);
  const auto state = [](int t) { return t == E5MA_FP32 || t == E5MA_BF16; };
  if (!state(param->dtype))
    return fail(E5MA_NOT_SUPPORTED, "e5ma_adam: param must be FP32 or BF16 (dtype %d)", (int)param->dtype);
  if (!state(exp_avg->dtype) || exp_avg_sq->dtype != exp_avg->dtype)
    return fail(E5MA_NOT_SUPPORTED, "e5ma_adam: exp_avg and exp_avg_sq must both be FP32 or both BF16 (dtypes %d, %d)",
                (int)exp_avg->dtype, (int)exp_avg_sq->dtype);
  if (grad->dtype < E5MA_BF16 || grad->dtype > E5MA_FP32)
    return fail(E5MA_NOT_SUPPORTED, "e5ma_adam: grad must be FP32, BF16 or FP16 (dtype %d)", (int)grad->dtype);
  if (param_fp8 && param_fp8->data && !is_fp8(param_fp8->dtype))
    return fail(E5MA_INVALID_VALUE, "e5ma_adam: param_fp8 must have dtype E5MA_E4M3 or E5MA_E5M2 (dtype %d)",
                (int)param_fp8->dtype);
  if (param_fp8 && param_fp8->data && param_fp8->scaling != E5MA_SCALING_TENSOR)
    return fail(E5MA_INVALID_VALUE, "e5ma_adam: param_fp8 takes per-tensor scaling only");
  if (count == 0) return E5MA_OK;
  int dev = 0;
  if (e5ma_status st = e5ma::check_device(&dev)) return st;
  // scalars formed in double and rounded to FP32 once (reference src/adamw_e5m2effma.cu:150-157)
  e5ma::AdamScalars a;
  a.lr = cfg->lr;
  a.beta1 = cfg->beta1;
  a.beta2 = cfg->beta2;
  a.eps = cfg->eps;
  a.wd = cfg->weight_decay;
  a.omb1 = (float)(1.0 - (double)cfg->beta1);
  a.omb2 = (float)(1.0 - (double)cfg->beta2);
  a.rbc1 = cfg->bias_correction ? (float)(1.0 / (1.0 - pow((double)cfg->beta1, cfg->step))) : 1.f;
  a.rbc2 = cfg->bias_correction ? (float)(1.0 / (1.0 - pow((double)cfg->beta2, cfg->step))) : 1.f;
  a.lr_wd = (float)((double)cfg->lr * cfg->weight_decay);
  a.gscale = cfg->grad_scale == 0.f ? 1.f : cfg->grad_scale;
  a.adamw = cfg->adamw;
  uint8_t *q = param_fp8 && param_fp8->data ? (uint8_t *)param_fp8->data : nullptr;
  const hipError_t err =
      e5ma::launch_adam(a, count, param->dtype, param->data, grad->dtype, grad->data, exp_avg->dtype, exp_avg->data,
                        exp_avg_sq->data, q ? (int)param_fp8->dtype : (int)E5MA_E4M3, q, q ? param_fp8->scale : nullptr,
                        q ? param_fp8->amax : nullptr, e5ma::device_info(dev).tune, stream);
  return e5ma::hip_status(err, "e5ma_adam: kernel launch");
}

// reference src/gemm_e5m2effma.cu:44-104
extern "C" e5ma_status e5ma_gemm(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                                 const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                                 const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                                 const e5ma_tensor *bias, hipStream_t stream) {
  e5ma::clear_error();
  const auto valid = [](const e5ma_tensor *t) { return valid_dtype(t->dtype); };
  const auto operand = [](int t) { return is_fp8(t) || t == E5MA_BF16 || t == E5MA_FP32; };
  const auto aligned16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
  const auto op_ok = [](int o) { return o == E5MA_OP_N || o == E5MA_OP_T; };
  if (!A || !B || !D || !A->data || !B->data || !D->data)
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: A, B, D or their data is NULL");
  if (!op_ok(transa) || !op_ok(transb))
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: transa / transb must be E5MA_OP_N or E5MA_OP_T");
  if (m < 0 || n < 0 || k < 0) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: negative size (m=%d n=%d k=%d)", m, n, k);
  if (!valid(D)) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: invalid D dtype %d", (int)D->dtype);
  if (!operand(A->dtype) || !operand(B->dtype))
    return fail(E5MA_NOT_SUPPORTED, "e5ma_gemm: A and B must be E5M2, E4M3, BF16 or FP32 (got dtypes %d, %d)",
                (int)A->dtype, (int)B->dtype);
  if (m == 0 || n == 0) return E5MA_OK;
  if (k % 16) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: k = %d is not a multiple of 16", k);
  if (lda % 16 || ldb % 16)
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: lda = %d / ldb = %d must be multiples of 16", lda, ldb);
  if (!aligned16(A->data) || !aligned16(B->data))
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: A and B must be 16-byte aligned");
  const bool a_kc = transa == E5MA_OP_T, b_kc = transb == E5MA_OP_N;
  if (lda < (a_kc ? k : m)) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: lda = %d < %d", lda, a_kc ? k : m);
  if (ldb < (b_kc ? k : n)) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: ldb = %d < %d", ldb, b_kc ? k : n);
  if (ldd < m) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: ldd = %d < m = %d", ldd, m);
  if (bias && bias->data && !valid(bias))
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: invalid bias dtype %d", (int)bias->dtype);
  if (beta != 0.f && C && C->data && !valid(C))
    return fail(E5MA_INVALID_VALUE, "e5ma_gemm: invalid C dtype %d", (int)C->dtype);
  if (beta != 0.f && C && C->data && ldc < m) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: ldc = %d < m = %d", ldc, m);
  const auto scaling_ok = [](const e5ma_tensor *t) {
    return t->scaling == E5MA_SCALING_TENSOR || t->scaling == E5MA_SCALING_OUTER;
  };
  if (!scaling_ok(A) || !scaling_ok(B)) return fail(E5MA_INVALID_VALUE, "e5ma_gemm: invalid scaling of A or B");
  for (const e5ma_tensor *t : {A, B})
    if (t->scaling == E5MA_SCALING_OUTER && (!is_fp8(t->dtype) || !t->scale_inv))
      return fail(E5MA_INVALID_VALUE, "e5ma_gemm: E5MA_SCALING_OUTER needs an FP8 operand with a scale_inv vector");
  for (const e5ma_tensor *t : {C, D, bias})
    if (t && t->scaling != E5MA_SCALING_TENSOR)
      return fail(E5MA_INVALID_VALUE, "e5ma_gemm: C, D and bias take per-tensor scaling only");
  int dev = 0;
  if (e5ma_status st = e5ma::check_device(&dev)) return st;
  const bool c_is_d = beta != 0.f && (!C || !C->data);  // TE "accumulate": D += ...

  e5ma::dev::Epilogue e;
  e.sa = is_fp8(A->dtype) ? A->scale_inv : nullptr;
  e.sb = is_fp8(B->dtype) ? B->scale_inv : nullptr;
  e.sa_vec = A->scaling == E5MA_SCALING_OUTER;
  e.sb_vec = B->scaling == E5MA_SCALING_OUTER;
  e.alpha = alpha;
  e.beta = beta;
  const e5ma_tensor *Cx = c_is_d ? D : C;
  e.c = beta != 0.f ? Cx->data : nullptr;
  e.ldc = beta != 0.f ? (c_is_d ? ldd : ldc) : 0;
  e.c_dtype = beta != 0.f ? (int)Cx->dtype : (int)E5MA_FP32;
  e.c_sinv = beta != 0.f && is_fp8(Cx->dtype) ? Cx->scale_inv : nullptr;
  e.d = D->data;
  e.ldd = ldd;
  e.d_dtype = D->dtype;
  e.d_scale = is_fp8(D->dtype) ? D->scale : nullptr;
  e.amax = D->amax;
  e.bias = bias && bias->data ? bias->data : nullptr;
  e.bias_dtype = bias ? (int)bias->dtype : (int)E5MA_FP32;

  const e5ma::DeviceInfo &di = e5ma::device_info(dev);
  const uint8_t *a = (const uint8_t *)A->data, *b = (const uint8_t *)B->data;
  const hipError_t err = n <= 8 && a_kc && b_kc && is_fp8(A->dtype)
                             ? e5ma::launch_gemv(A->dtype, B->dtype, a, lda, b, ldb, m, n, k, e, di, stream)
                             : e5ma::launch_gemm(A->dtype, B->dtype, a_kc, b_kc, a, lda, b, ldb, m, n, k, e, di, stream);
  return e5ma::hip_status(err, "e5ma_gemm: kernel launch");
}
