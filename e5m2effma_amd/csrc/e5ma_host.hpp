// e5ma_host.hpp -- internal host interface between the entry points (api.cpp, noalloc.hip) and the
// kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "e5m2effma.h"
#include "e5ma_device.hpp"

namespace e5ma {

// ---- status and the calling thread's message ----------------------------------------------------
// Every entry point opens a Call, which empties the thread's message; rules then run in order and the
// first broken one decides the status and the message (later rules are not evaluated).
class Call {
 public:
  Call();
  bool ok() const { return status_ == E5MA_OK; }
  e5ma_status status() const { return status_; }
  // a rule: when it does not hold (and no earlier rule failed), record status s and the message
  Call &need(bool holds, e5ma_status s, const char *fmt, ...) __attribute__((format(printf, 4, 5)));
  // a HIP result: hipSuccess, or E5MA_HIP_ERROR with "<what>: HIP error <n> (<name>): <text>"
  e5ma_status hip(hipError_t e, const char *what);

 private:
  e5ma_status status_ = E5MA_OK;
};
const char *thread_message();

// Launch choices that depend on the device.  The defaults were measured on MI355X (256 CUs);
// e5ma_tuned.h, written by the tuner (e5m2effma_amd/tune/tune.cpp, which times the candidates on the
// device), holds the entries per (architecture, CU count), and a device without an entry runs these
// defaults.  The grid caps of the streaming kernels never change results (every element is computed
// alone, and amax is an exact maximum).  splitk_div does: it decides whether a small grid splits K
// (only where the caller supplies a workspace, e5ma_gemm_ex / e5ma_gemm_noalloc), and a split sums the
// products in another order, so the result may differ in the last bits while staying inside the
// GEMM's accumulation bound.
struct Tuning {
  int splitk_div = 4;          // split K when tiles * splitk_div <= CUs (0: never)
  int cast_grid = 8192;        // block cap of the grid-stride cast and quantize kernels
  int adam_grid_bf16 = 65536;  // block cap of the Adam kernel with BF16 parameters
  int adam_grid_fp32 = 8192;   // ... with FP32 parameters
  int quant_grid = 8192;       // block cap of the per-tensor quantize's amax pass (its cast pass: cast_grid)
  int tail_half = 0;           // FP8 GEMM: 1 runs a last round of at most CUs / 2 tiles as 256 x 128 half tiles
                               // (the same bits either way; measured slower on the MI355X, so 0 there)
  int gemv_rows = 2;           // GEMV n = 1 with a BF16 / FP8 x: rows per wave (1, 2 or 4; 8 / rows 16-byte chunks
                               // per lane and batch).  Every choice sums each row in the same order: the same bits
};

struct DeviceInfo {
  int cus = 0;          // compute units
  int xcds = 8;         // accelerator complex dies (L2 domains)
  bool supported = false;
  char arch[64] = {0};
  Tuning tune;          // e5ma_tuned.h's entry for (arch, cus), or the defaults
};
// Properties of device dev (cached per device, dev < kMaxDevices); resolve_device() reads the current
// device and reports an unsupported one or an index beyond the cache.
constexpr int kMaxDevices = 64;
const DeviceInfo &device_info(int dev);
e5ma_status resolve_device(Call &call, int *dev_out);

// ---- kernel launchers (each returns the launch status) -----------------------------------------
hipError_t launch_cast(int tin, int tout, const void *src, void *dst, size_t count, const float *sinv,
                       const float *qscale, float *amax, const Tuning &t, hipStream_t s);

// Float8Tensor.from_float's quantization (include/e5m2effma_ext.h): per tensor (two passes) or per row.
hipError_t launch_quantize(int tin, int tout, const void *src, void *dst, size_t rows, size_t cols, const float *sinv,
                           float qmax, bool per_row, float *scale_inv, float *amax, const Tuning &t, hipStream_t s);

// The per-element coefficients of one Adam / AdamW step (include/e5m2effma.h):
//   g = grad * grad_mul;  Adam: g = fma(l2, p, g)
//   m = fma(b1, m, c1 * g);  v = fma(b2, v, c2 * (g * g))
//   u = (m * corr1) / (sqrt(v * corr2) + eps)
//   AdamW: p = fma(-decay, p, p);  then p = fma(-lr, u, p)
struct AdamCoefficients {
  float grad_mul;
  float l2;            // weight_decay, the gradient's L2 term (Adam)
  float b1, c1;        // beta1, 1 - beta1
  float b2, c2;        // beta2, 1 - beta2
  float corr1, corr2;  // bias corrections 1 / (1 - beta^step), or 1
  float eps;
  float decay;         // lr * weight_decay, the decoupled decay (AdamW)
  float lr;
  int decoupled;       // 1: AdamW, 0: Adam
};
hipError_t launch_adam(const AdamCoefficients &a, size_t count, int pt, void *p, int gt, const void *g, int mt,
                       void *m, void *v, int qt, uint8_t *q, const float *qscale, float *amax, const Tuning &t,
                       hipStream_t s);

// GEMV: D = epilogue(A^T x) for an FP8 A stored K-contiguous (transa = T) and n <= 8 K-contiguous
// columns of B (transb = N).
hipError_t launch_gemv(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m,
                       int n, int k, const dev::Epilogue &e, const DeviceInfo &di, hipStream_t s);

// Device memory a GEMM may use for split-K partials (none: never split).  Caller-owned
// (e5ma_gemm_ex) or the library's fixed per-device scratch (e5ma_gemm_noalloc); 256-byte aligned.
struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};
// the most split-K workspace any GEMM asks for
constexpr size_t kMaxWorkspace = (size_t)64 << 20;

// Tiled GEMM on the matrix cores.  akc / bkc: operand stored K-contiguous.
hipError_t launch_gemm(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                       long long ldb, int m, int n, int k, const dev::Epilogue &e, const DeviceInfo &di,
                       const Workspace &ws, hipStream_t s);
// the split-K workspace the same call would use given unlimited bytes (0: it never splits)
size_t gemm_workspace_bytes(int at, int bt, bool akc, bool bkc, int m, int n, int k, long long lda, long long ldb,
                            const DeviceInfo &di);

// ---- e5ma_gemm's request, shared by every GEMM entry point (api.cpp) ----------------------------
// Where a GEMM's split-K workspace comes from: memory the caller gave (or none), or, when per_device is
// set, a function that returns device dev's memory once the arguments have passed their rules and dev
// is the current device (it reports a failure through call).
// A per-device workspace has a fixed capacity: a call whose split-K partials would need more is
// rejected (the caller's workspace of e5ma_gemm_ex instead limits the split count).
struct WorkspaceSource {
  Workspace given;
  Workspace (*per_device)(int dev, Call &call) = nullptr;
};
e5ma_status gemm_entry(const char *name, e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                       const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                       const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd, const e5ma_tensor *bias,
                       const WorkspaceSource &src, hipStream_t stream);

}  // namespace e5ma
