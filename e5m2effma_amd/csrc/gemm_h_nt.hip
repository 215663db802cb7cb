// gemm_h_nt.hip -- instances of the BF16-matrix-core GEMM for transa, transb = n, t (A M-contiguous, B N-contiguous).
#include "gemm_h_kernel.hpp"

namespace e5ma {
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nt) { return hk::launch_layout<false, false>(at, bt, A, lda, B, ldb, m, n, k, splits, cus, e, s); }
}  // namespace e5ma
