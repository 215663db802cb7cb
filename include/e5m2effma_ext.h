/* e5m2effma_ext.h -- an entry point of the MI355X library beyond the reference's C ABI.
 *
 * e5ma_quantize has no counterpart in the reference's C interface (include/e5m2effma.h there exports
 * gemm, cast, adam and the status functions).  It replaces the step the reference composes from
 * torch operations and e5ma_cast in Float8Tensor.from_float
 * (binds/python/e5m2effma/tensor.py:52-74): FP8 codes whose scale comes from the data's own amax.
 * Same status codes and thread-local message as the other entry points (e5ma_last_error).
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

#ifdef __cplusplus
}
#endif
#endif /* E5M2EFFMA_EXT_H */
