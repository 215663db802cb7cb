// gemm.hip -- kernel choice for the tiled path of e5ma_gemm (reference src/gemm_e5m2effma.cu:18-39).
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {

hipError_t launch_gemm(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                       long long ldb, int m, int n, int k, const dev::Epilogue &e, const DeviceInfo &,
                       hipStream_t s) {
  if (gemm_f8_applies(at, bt, akc, bkc, m, n, k)) return launch_gemm_f8(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  if (gemm_h_applies(at, bt, akc, bkc, m, n, k)) return launch_gemm_h(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  return launch_gemm_generic(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
}

}  // namespace e5ma
