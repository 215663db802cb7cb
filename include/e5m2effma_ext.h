/* e5m2effma_ext.h -- entry points of the MI355X library beyond the reference's C ABI.
 *
 * None of these has a counterpart in the reference's C interface (include/e5m2effma.h there exports
 * gemm, cast, adam and the status functions).  Same status codes and thread-local message as the other
 * entry points (e5ma_last_error).
 *   e5ma_quantize             replaces the step the reference composes from torch operations and
 *                             e5ma_cast in Float8Tensor.from_float (binds/python/e5m2effma/tensor.py:52-74)
 *   e5ma_gemm_ex              e5ma_gemm with a caller-owned workspace for split-K on small grids
 *   e5ma_gemm_workspace_size  the workspace e5ma_gemm_ex uses for a shape
 *   e5ma_gemm_noalloc         e5ma_gemm_ex on the library's fixed per-device scratch: allocates nothing
 */
#ifndef E5M2EFFMA_EXT_H
#define E5M2EFFMA_EXT_H

#include "e5m2effma.h"

#ifdef __cplusplus
extern "C" {
#endif

/* src: rows x cols elements, row-major (row r starts at element r * cols), any dtype; an FP8 source
 * is decoded times src->scale_inv (NULL = 1).  dst: E5MA_E4M3 or E5MA_E5M2, same element layout;
 * dst->scaling selects one scale for the whole tensor (E5MA_SCALING_TENSOR) or one per row
 * (E5MA_SCALING_OUTER); dst->scale and dst->amax are not used.  Per tensor, or per row:
 *   amax  = max |v|                        (a NaN anywhere makes it NaN, as torch's amax does)
 *   scale = fl(fl(1 / max(amax, 1e-12)) * qmax)     (torch's `qmax / amax` is reciprocal() * qmax)
 *   codes = RNE satfinite of v * scale     (e5ma_cast's encoder; a NaN becomes 0x7F)
 *   scale_inv[g] = 1 / scale  (written; device, 1 or rows floats)
 *   amax_out[g]  = amax       (optional, written; device, 1 or rows floats)
 * qmax is the value the amax maps to: the format's largest finite value (57344 for E5M2, 448 for
 * E4M3) times a margin, rounded to FP32 by the caller.  Per tensor, scale_inv[0] also serves as the
 * reduction word while the call runs (two passes over src); per row (rows < 2^24), each row of at
 * most 16384 elements (cols a multiple of 16, 16-byte aligned buffers) is read once. */
e5ma_status e5ma_quantize(const e5ma_tensor *src, const e5ma_tensor *dst, size_t rows, size_t cols,
                          float qmax, float *scale_inv, float *amax_out, hipStream_t stream);

/* e5ma_gemm (include/e5m2effma.h: same arguments, rules, semantics and messages, prefixed
 * "e5ma_gemm_ex") with device memory the caller owns for split-K.  e5ma_gemm itself allocates and uses
 * no device memory beyond its arguments, so an output of few 256 x 256 tiles occupies few of the 256
 * compute units.  Given a workspace, such an output (at most 1/4 of the CUs' worth of tiles by default)
 * splits K over more blocks: FP32 partials in the workspace, summed in split order by a second kernel
 * on the same stream (deterministic for a given device, shape and workspace size).  Its result stays
 * inside the accumulation bound of e5ma_gemm but may differ from e5ma_gemm's in the last bits, and
 * whether a shape splits depends on the device's CU count and tuning.  A workspace smaller than
 * e5ma_gemm_workspace_size()'s gives fewer splits, a NULL / 0-byte one none (then the call is e5ma_gemm).
 * workspace: device memory, 256-byte aligned, used in stream order and free again when the call's work
 * on `stream` has finished; the library keeps no reference to it.  Calls that share one workspace must
 * be ordered (one stream, or events). */
e5ma_status e5ma_gemm_ex(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                         const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                         const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                         const e5ma_tensor *bias, void *workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* The workspace e5ma_gemm_ex would use for this shape on the current device, in *bytes (0: it never
 * splits; at most 64 MiB).  lda / ldb as for the GEMM call. */
e5ma_status e5ma_gemm_workspace_size(e5ma_op transa, e5ma_op transb, int m, int n, int k,
                                     e5ma_dtype a_dtype, int lda, e5ma_dtype b_dtype, int ldb,
                                     size_t *bytes);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  e5ma_gemm_ex with the library's own
 * scratch as the workspace: a fixed 64 MiB per device (the largest workspace any GEMM asks for), a
 * file-scope device array reserved when the library loads on a device and held until the process ends.
 * The call allocates nothing.  Same results as e5ma_gemm_ex given e5ma_gemm_workspace_size()'s bytes; a
 * call whose split-K partials would need more than the scratch is rejected with E5MA_INVALID_VALUE (none
 * does with 64 MiB).  Every call on a device shares that device's scratch: calls whose work overlaps on
 * one device (unordered streams) race on it and must not be issued. */
e5ma_status e5ma_gemm_noalloc(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                              const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                              const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                              const e5ma_tensor *bias, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* E5M2EFFMA_EXT_H */
