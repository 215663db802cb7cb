// e5ma_host.hpp -- internal host interface between the C ABI (api.cpp) and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "e5m2effma.h"
#include "e5ma_device.hpp"

namespace e5ma {

// thread-local error message (reference src/e5m2effma.cu:11-24)
void clear_error();
e5ma_status fail(e5ma_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
e5ma_status hip_status(hipError_t e, const char *what);

// Launch choices that depend on the device, not on correctness: every value gives identical results.
// The defaults were measured on MI355X (256 CUs); e5ma_tuned.h, written by the tuner
// (e5m2effma_amd/tune/tune.cpp, which times the candidates on the device), holds the entries per
// (architecture, CU count), and a device without an entry runs these defaults.
struct Tuning {
  int splitk_div = 4;          // split K when tiles * splitk_div <= CUs (0: never)
  int cast_grid = 8192;        // block cap of the grid-stride cast and quantize kernels
  int adam_grid_bf16 = 65536;  // block cap of the Adam kernel with BF16 parameters
  int adam_grid_fp32 = 8192;   // ... with FP32 parameters
  int quant_grid = 8192;       // block cap of the per-tensor quantize's amax pass (its cast pass: cast_grid)
};

struct DeviceInfo {
  int cus = 0;          // compute units
  int xcds = 8;         // accelerator complex dies (L2 domains)
  bool supported = false;
  char arch[64] = {0};
  Tuning tune;          // e5ma_tuned.h's entry for (arch, cus), or the defaults
  // The library's own stream-ordered memory pool on this device (null if unavailable): split-K
  // workspaces come from it.  Its release threshold is unlimited, so a freed workspace stays mapped
  // and the next call reuses it, and the process's default pool keeps its own settings.
  hipMemPool_t pool = nullptr;
};
// Current device's properties (cached per device); check_device() reports an unsupported device.
const DeviceInfo &device_info(int dev);
e5ma_status check_device(int *dev_out = nullptr);

// ---- kernel launchers (each returns the launch status) -----------------------------------------
hipError_t launch_cast(int tin, int tout, const void *src, void *dst, size_t count, const float *sinv,
                       const float *qscale, float *amax, const Tuning &t, hipStream_t s);

// Float8Tensor.from_float's quantization (include/e5m2effma_ext.h): per tensor (two passes) or per row.
hipError_t launch_quantize(int tin, int tout, const void *src, void *dst, size_t rows, size_t cols, const float *sinv,
                           float qmax, bool per_row, float *scale_inv, float *amax, const Tuning &t, hipStream_t s);

struct AdamScalars {
  float lr, beta1, beta2, omb1, omb2, rbc1, rbc2, eps, lr_wd, wd, gscale;
  int adamw;
};
hipError_t launch_adam(const AdamScalars &a, size_t count, int pt, void *p, int gt, const void *g, int mt,
                       void *m, void *v, int qt, uint8_t *q, const float *qscale, float *amax, const Tuning &t,
                       hipStream_t s);

// GEMV: D = epilogue(A^T x) for an FP8 A stored K-contiguous (transa = T) and n <= 8 K-contiguous
// columns of B (transb = N).
hipError_t launch_gemv(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m,
                       int n, int k, const dev::Epilogue &e, const DeviceInfo &di, hipStream_t s);

// Tiled GEMM on the matrix cores.  akc / bkc: operand stored K-contiguous.
hipError_t launch_gemm(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                       long long ldb, int m, int n, int k, const dev::Epilogue &e, const DeviceInfo &di,
                       hipStream_t s);

}  // namespace e5ma
