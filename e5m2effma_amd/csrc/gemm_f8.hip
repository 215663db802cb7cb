// gemm_f8.hip -- when the fast FP8 GEMM applies, and its layout dispatch (the kernel is in
// gemm_f8_kernel.hpp; one translation unit per layout pair holds its instances).
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {

namespace {
constexpr int kRound = 256;  // the K loop runs whole rings (4 x 64 or 2 x 128 K bytes)
}

bool gemm_f8_applies(int at, int bt, bool akc, bool bkc, int m, int n, int k, long long lda, long long ldb) {
  // at least 2 rounds; an M / N-contiguous operand is loaded in whole 16-byte chunks of its rows, so its
  // m (n) is a multiple of 16; the loads' 32-bit per-lane offsets need lda, ldb <= kMaxLd bytes
  return is_fp8(at) && is_fp8(bt) && k % kRound == 0 && k >= 2 * kRound && gemm::mode_of(at, bt, k) == gemm::kModeF8 &&
         m > 0 && n > 0 && (akc || m % 16 == 0) && (bkc || n % 16 == 0) && lda <= kMaxLd && ldb <= kMaxLd;
}

hipError_t launch_gemm_f8(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                          long long ldb, int m, int n, int k, int splits, int cus, int tail_half, const dev::Epilogue &e,
                          hipStream_t s) {
  if (akc) return (bkc ? launch_gemm_f8_tn : launch_gemm_f8_tt)(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s);
  return (bkc ? launch_gemm_f8_nn : launch_gemm_f8_nt)(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s);
}

int gemm_f8_round() { return kRound; }

}  // namespace e5ma
