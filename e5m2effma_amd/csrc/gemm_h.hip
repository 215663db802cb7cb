// gemm_h.hip -- when the fast BF16-matrix-core GEMM applies, and its layout dispatch (the kernel is in
// gemm_h_kernel.hpp; one translation unit per layout pair holds its instances).
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {

int gemm_h_round(int bt) { return 4 * (bt == E5MA_BF16 ? 32 : 64); }

bool gemm_h_applies(int at, int bt, bool akc, bool bkc, int m, int n, int k) {
  // FP8 A; FP8 B in any layout or a K-contiguous BF16 B; whole rounds of the 4-slot ring of KS-k stages
  // (KS = 64, or 32 with a BF16 B), at least 2 rounds; an M / N-contiguous operand needs m (n) a
  // multiple of 16
  if (!is_fp8(at) || !(is_fp8(bt) || (bt == E5MA_BF16 && bkc))) return false;
  if (gemm::mode_of(at, bt, k) != gemm::kModeH) return false;
  const int round = gemm_h_round(bt);
  return k % round == 0 && k >= 2 * round && m > 0 && n > 0 && (akc || m % 16 == 0) && (bkc || n % 16 == 0);
}

hipError_t launch_gemm_h(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                         long long ldb, int m, int n, int k, int splits, int cus, int tail_half, const dev::Epilogue &e,
                         hipStream_t s) {
  // (tail_half: the BF16-core kernel runs whole tiles only; cus: its persistent grid)
  if (bt == E5MA_BF16)
    return (akc ? launch_gemm_h_tn_bf16 : launch_gemm_h_nn_bf16)(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s);
  if (akc) return (bkc ? launch_gemm_h_tn : launch_gemm_h_tt)(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s);
  return (bkc ? launch_gemm_h_nn : launch_gemm_h_nt)(at, bt, A, lda, B, ldb, m, n, k, splits, cus, tail_half, e, s);
}

}  // namespace e5ma
