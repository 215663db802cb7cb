// gemm_h_nn_bf16.hip -- instances of the BF16-matrix-core GEMM for an FP8 A times a K-contiguous BF16 B,
// transa, transb = n, n (A M-contiguous).
#include "gemm_h_kernel.hpp"

namespace e5ma {
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nn_bf16) { return hk::launch_layout_bf16<false>(at, bt, A, lda, B, ldb, m, n, k, splits, cus, e, s); }
}  // namespace e5ma
