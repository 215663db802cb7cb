// gemm_f8_nn.hip -- instances of the fast FP8 GEMM for transa, transb = n, n (A M-contiguous, B K-contiguous).
#include "gemm_f8_kernel.hpp"

namespace e5ma {
E5MA_F8_LAYOUT_DECL(launch_gemm_f8_nn) { return f8k::launch_layout<false, true>(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s); }
}  // namespace e5ma
