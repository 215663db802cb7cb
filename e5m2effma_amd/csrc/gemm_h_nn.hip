// gemm_h_nn.hip -- instances of the BF16-matrix-core GEMM for transa, transb = n, n (A M-contiguous, B K-contiguous).
#include "gemm_h_kernel.hpp"

namespace e5ma {
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nn) { return hk::launch_layout<false, true>(at, bt, A, lda, B, ldb, m, n, k, splits, cus, e, s); }
}  // namespace e5ma
