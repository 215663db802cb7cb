/* e5m2effma.h -- C ABI of the MI355X (gfx950) FP8 compute library.
 *
 * Drop-in for the reference interface /root/reference/include/e5m2effma.h (E5M2EffMA 0.2.0):
 * every enum value, struct layout (LP64: e5ma_tensor is 48 bytes, e5ma_adam_config 36 bytes) and
 * function signature is identical; the stream slot is a hipStream_t (pointer-sized, so the argument
 * is ABI-identical to the reference's cudaStream_t).
 *
 * GEMM (column-major, cuBLASLt / Transformer Engine semantics):
 *
 *     D = alpha * (sa * sb) * op(A) * op(B) + bias + beta * C          D, C: m x n
 *
 *   op(A) m x k: transa = T -> A stored k x m (lda >= k, K-contiguous), N -> m x k (lda >= m).
 *   op(B) k x n: transb = N -> B stored k x n (ldb >= k, K-contiguous), T -> n x k (ldb >= n).
 *   A, B in {E5M2, E4M3, BF16, FP32}, any pairing.  sa / sb: scale_inv of FP8 operands (NULL = 1),
 *   one per tensor or, with E5MA_SCALING_OUTER, one per row of op(A) (m floats) / column of op(B)
 *   (n floats).  bias: length m, any dtype.  C: any dtype (FP8 C dequantized by C->scale_inv), may
 *   alias D; C == NULL with beta != 0 accumulates into D (TE "accumulate", e.g. FP32 main_grad).
 *
 *   Arithmetic on gfx950: FP8 x FP8 on the f8f6f4 matrix cores (products exact, FP32 accumulation);
 *   FP8 x BF16 and BF16 x BF16 with FP8 upcast exactly to BF16 on the BF16 matrix cores; anything
 *   with an FP32 operand on the FP32 matrix cores.  The accumulation order is that of the matrix
 *   cores (not the reference's ascending-k FFMA chain); every result satisfies
 *   |acc - exact| <= 2 * k * 2^-24 * sum|a*b|.
 *   Epilogue, in FP32, in this order:  v = acc * s (s = (alpha * sa[i]) * sb[j]);  v = v + bias[i];
 *   v = fma(beta, C[i, j] * csinv, v);  amax = max(amax, |v|) (NaN ignored);  D = convert(v)
 *   (BF16 / FP16 / FP32: round to nearest even, NaN -> 0x7FC0 for BF16; FP8: RNE satfinite of
 *   v * D->scale, every NaN -> 0x7F).
 *   Routing: n <= 8, transa = T, transb = N and an FP8 A run the bandwidth-bound GEMV kernel.
 *
 *   Requirements: A and B 16-byte aligned; k, lda, ldb multiples of 16; ldd >= m (ldc >= m when C
 *   is read).  FP8 GEMM operands are decoded as OCP FP8 by the matrix cores: an E5M2 Inf / NaN code
 *   or the E4M3 NaN code in A or B propagates as Inf / NaN (the reference reads them as finite
 *   numbers; both call them outside the contract).
 */
#ifndef E5M2EFFMA_H
#define E5M2EFFMA_H

#define E5M2EFFMA_VERSION "0.2.0"

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/e5m2effma.h:54 */
typedef enum { E5MA_E4M3 = 0, E5MA_BF16 = 1, E5MA_FP16 = 2, E5MA_FP32 = 3, E5MA_E5M2 = 4 } e5ma_dtype;
/* reference include/e5m2effma.h:55 */
typedef enum { E5MA_OP_N = 0, E5MA_OP_T = 1 } e5ma_op;
/* reference include/e5m2effma.h:56.  Value 3 reports a HIP runtime / device failure; the
 * reference's name E5MA_CUDA_ERROR is kept so that callers written against it compile unchanged. */
typedef enum {
  E5MA_OK = 0,
  E5MA_INVALID_VALUE = 1,
  E5MA_NOT_SUPPORTED = 2,
  E5MA_CUDA_ERROR = 3,
  E5MA_HIP_ERROR = 3
} e5ma_status;
/* reference include/e5m2effma.h:59: scale_inv of an FP8 GEMM operand per tensor, or per outer index */
typedef enum { E5MA_SCALING_TENSOR = 0, E5MA_SCALING_OUTER = 1 } e5ma_scaling;

/* reference include/e5m2effma.h:61-70 */
typedef struct {
  void *data;              /* device pointer */
  e5ma_dtype dtype;
  const float *scale_inv;  /* FP8 input: dequantization factor (device, 1 float), NULL = 1 */
  const float *scale;      /* FP8 output: quantization factor (device, 1 float), NULL = 1 */
  float *amax;             /* optional: max |v| before quantization, max-reduced into *amax */
  e5ma_scaling scaling;    /* FP8 GEMM operands only: E5MA_SCALING_OUTER = scale_inv vector */
} e5ma_tensor;

/* Replaces reference e5ma_gemm (include/e5m2effma.h:73-76, src/gemm_e5m2effma.cu:44-104).  Like the
 * reference it allocates and uses no device memory beyond its arguments, and it gives the same bits on
 * every MI355X for the same inputs (e5ma_gemm_ex in e5m2effma_ext.h adds split-K with a caller-owned
 * workspace). */
e5ma_status e5ma_gemm(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                      const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                      const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                      const e5ma_tensor *bias, hipStream_t stream);

/* Replaces reference e5ma_cast (include/e5m2effma.h:78-81, src/e5m2effma.cu:85-101).
 * v = src * src.scale_inv (FP8 source; Inf / NaN codes decode to Inf / NaN); amax = max |v|;
 * dst = convert(v) (FP8 destination: RNE satfinite of v * dst.scale). */
e5ma_status e5ma_cast(const e5ma_tensor *src, const e5ma_tensor *dst, size_t count, hipStream_t stream);

/* reference include/e5m2effma.h:95-101 */
typedef struct {
  float lr, beta1, beta2, eps, weight_decay;
  int step;             /* 1-based */
  int adamw;            /* 1: decoupled weight decay; 0: L2 term added to the gradient */
  int bias_correction;  /* 1: Adam bias correction */
  float grad_scale;     /* gradient multiplier (0 is treated as 1) */
} e5ma_adam_config;

/* Replaces reference e5ma_adam (include/e5m2effma.h:103-106, src/adamw_e5m2effma.cu:125-168).
 * Per element, in FP32:
 *   g = grad * grad_scale;  if (!adamw) g = fma(weight_decay, p, g)
 *   m = fma(beta1, m, (1 - beta1) * g);   v = fma(beta2, v, (1 - beta2) * (g * g))
 *   u = (m * rbc1) / (sqrt(v * rbc2) + eps)     (correctly rounded / and sqrt)
 *   if (adamw) p = fma(-(lr * weight_decay), p, p);   p = fma(-lr, u, p)
 * 1 - beta, rbc = 1 / (1 - beta^step) and lr * weight_decay are formed in double and rounded to
 * FP32 once.  param FP32 / BF16; grad FP32 / BF16 / FP16; exp_avg, exp_avg_sq both FP32 or both
 * BF16; param_fp8 (optional) E4M3 / E5M2 copy of the updated weights quantized with its scale,
 * its amax receiving max |p|. */
e5ma_status e5ma_adam(const e5ma_adam_config *cfg, size_t count, const e5ma_tensor *param,
                      const e5ma_tensor *grad, const e5ma_tensor *exp_avg,
                      const e5ma_tensor *exp_avg_sq, const e5ma_tensor *param_fp8,
                      hipStream_t stream);

/* Replaces reference e5ma_status_string (include/e5m2effma.h:108, src/e5m2effma.cu:103-111). */
const char *e5ma_status_string(e5ma_status status);

/* Replaces reference e5ma_last_error (include/e5m2effma.h:110-112, src/e5m2effma.cu:83): the most
 * recent failure of an e5ma_* call on the calling thread, "" after a successful call. */
const char *e5ma_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* E5M2EFFMA_H */
