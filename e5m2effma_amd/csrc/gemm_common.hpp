// gemm_common.hpp -- types and operand helpers shared by the matrix-core GEMM kernels.
#pragma once
#include "e5ma_device.hpp"

namespace e5ma {
namespace gemm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Arithmetic modes: F8 = FP8 x FP8 on the f8f6f4 matrix cores; H = BF16 matrix cores (FP8 upcast
// exactly to BF16); S = FP32 matrix cores (everything decoded exactly to FP32).
constexpr int kModeF8 = 0, kModeH = 1, kModeS = 2;

// Accuracy of the FP8 matrix cores, and why F8 mode needs k >= kF8MinK.
// Measured on gfx950 (v_mfma_scale_f32_32x32x64_f8f6f4 and the older v_mfma_f32_32x32x16_{fp8,bf8}
// behave alike): the products of each group of 8 consecutive k are exact, but each is truncated
// toward zero to a multiple of 2^(E - 13), E the exponent of the group's largest product; partial
// sums of 16 products then enter the FP32 accumulator with round-toward-zero.  The error of one
// output is therefore below 7 * 2^-13 * sum_g max_g|p| + (k / 16) * 2^-23 * sum|p|
//                      <= (7 * 2^-13 + k * 2^-27) * sum|a*b|,
// which stays inside the library's contract |acc - exact| <= 2 * k * 2^-24 * sum|a*b| exactly when
// k >= 7 * 2^14 / 15 (about 7646).  Shorter reductions run in H mode: FP8 values are exact in BF16,
// BF16 products are exact in FP32, and the BF16 matrix cores accumulate in FP32 (measured error
// about 4 * 2^-24 * sum|a*b| per 64 k).
constexpr int kF8MinK = 8192;
__host__ __device__ constexpr int mode_of(int a, int b, int k) {
  return a == E5MA_FP32 || b == E5MA_FP32 ? kModeS : (is_fp8(a) && is_fp8(b) && k >= kF8MinK ? kModeF8 : kModeH);
}
// E8M0 block scale 2^0: the scaled f8f6f4 MFMA then computes the plain product
constexpr int kNeutralScale = 127;
// f8f6f4 operand format selector (cbsz for A, blgp for B): 0 = E4M3, 1 = E5M2
template <int T> constexpr int kMfmaFmt = T == E5MA_E5M2 ? 1 : 0;

// GEMM operand element idx of dtype T as an exact FP32 value.  FP8 codes decode as OCP values, the
// way the matrix cores read them (Inf / NaN codes propagate).
template <int T> __device__ __forceinline__ float operand_value(const uint8_t *base, long long idx) {
  if constexpr (T == E5MA_E5M2) return dev::e5m2_value(base[idx]);
  else if constexpr (T == E5MA_E4M3) return dev::e4m3_value(base[idx]);
  else if constexpr (T == E5MA_BF16) return dev::bf16_value(((const uint16_t *)base)[idx]);
  else return ((const float *)base)[idx];
}

// 4 FP8 codes of a dword -> 4 exact FP32 values (hardware packed converts, OCP decoding)
template <int T> __device__ __forceinline__ void decode4(uint32_t w, float *v) {
  if constexpr (T == E5MA_E5M2) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
    v[0] = lo[0]; v[1] = lo[1]; v[2] = hi[0]; v[3] = hi[1];
  } else {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    v[0] = lo[0]; v[1] = lo[1]; v[2] = hi[0]; v[3] = hi[1];
  }
}

// N (8 or 16) consecutive operand values of dtype T at p (aligned to N * bytes(T)) -> FP32
template <int T, int N> __device__ __forceinline__ void load_group(const uint8_t *p, float *v) {
  if constexpr (is_fp8(T)) {
    if constexpr (N == 16) {
      const uint4 q = *(const uint4 *)p;
      decode4<T>(q.x, v); decode4<T>(q.y, v + 4); decode4<T>(q.z, v + 8); decode4<T>(q.w, v + 12);
    } else {
      const uint2 q = *(const uint2 *)p;
      decode4<T>(q.x, v); decode4<T>(q.y, v + 4);
    }
  } else if constexpr (T == E5MA_BF16) {
#pragma unroll
    for (int h = 0; h < N / 8; ++h) {
      const uint4 q = ((const uint4 *)p)[h];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * h + 2 * e] = __uint_as_float(w[e] << 16);
        v[8 * h + 2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < N / 4; ++h) {
      const float4 q = ((const float4 *)p)[h];
      v[4 * h] = q.x; v[4 * h + 1] = q.y; v[4 * h + 2] = q.z; v[4 * h + 3] = q.w;
    }
  }
}

// Applies the epilogue to a staged block of accumulators: stage[jl * ld + il] holds output
// (i0 + il, j0 + jl), il < rows, jl < cols.  Consecutive threads take consecutive il, so D, C and bias
// accesses run along the contiguous dimension.  Deliberately not unrolled: the dtype dispatch of the
// epilogue is large, and one copy of it serves every kernel.  Returns the thread's max |value|.
template <int THREADS>
__device__ __attribute__((noinline)) float epilogue_block(const dev::Epilogue &e, const float *stage, int ld, int rows,
                                                          int cols, int i0, int j0, int m, int n) {
  const dev::EpiState st = dev::epi_begin(e);
  float mx = 0.f;
  const int total = rows * cols;
#pragma unroll 1
  for (int idx = threadIdx.x; idx < total; idx += THREADS) {
    const int il = idx % rows, jl = idx / rows;
    const int i = i0 + il, j = j0 + jl;
    if (i < m && j < n) {
      const float v = dev::epi_value(e, st, i, j, stage[jl * ld + il]);
      dev::store_any(e.d_dtype, e.d, (size_t)j * e.ldd + i, v, st.qscale);
      mx = dev::amax_fold(mx, v);
    }
  }
  return mx;
}

}  // namespace gemm

// largest leading dimension (bytes) of an operand of the fast kernels: their direct-to-LDS loads
// address a stage as a wave-uniform base plus 32-bit per-lane offsets of up to 255 rows
constexpr long long kMaxLd = 1LL << 24;

// fast FP8 x FP8 path (gemm_f8.hip), any operand layout; akc / bkc: A / B K-contiguous
bool gemm_f8_applies(int at, int bt, bool akc, bool bkc, int m, int n, int k, long long lda, long long ldb);
hipError_t launch_gemm_f8(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                          long long ldb, int m, int n, int k, int splits, int cus, int tail_half, const dev::Epilogue &e,
                          hipStream_t s);
// its instances, one translation unit per layout pair, named for (transa, transb):
// tn = both K-contiguous, nn = A M-contiguous, nt = both M / N-contiguous, tt = B N-contiguous.
// splits > 1: k is split into that many equal parts (each a multiple of the kernel's ring round), and
// e describes FP32 partial outputs, split s at e.d + s * e.ldd * n floats.  FP8 kernel: cus > 0 caps the
// grid at that many blocks, each taking every cus-th tile (persistent); tail_half (splits = 1): a last round
// of at most cus / 2 tiles runs as half tiles.  The results are the same bits either way.
#define E5MA_F8_LAYOUT_DECL(NAME)                                                                                   \
  hipError_t NAME(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n, \
                  int k, int splits, int cus, int tail_half, const dev::Epilogue &e, hipStream_t s)
E5MA_F8_LAYOUT_DECL(launch_gemm_f8_tn);
E5MA_F8_LAYOUT_DECL(launch_gemm_f8_nn);
E5MA_F8_LAYOUT_DECL(launch_gemm_f8_nt);
E5MA_F8_LAYOUT_DECL(launch_gemm_f8_tt);
// fast BF16-matrix-core path (gemm_h.hip): FP8 A x FP8 B (k < kF8MinK) or x K-contiguous BF16 B
bool gemm_h_applies(int at, int bt, bool akc, bool bkc, int m, int n, int k);
hipError_t launch_gemm_h(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                         long long ldb, int m, int n, int k, int splits, int cus, int tail_half, const dev::Epilogue &e,
                         hipStream_t s);
// K of one ring round of the fast kernels (a split's K is a multiple of it, at least two of them)
int gemm_f8_round();
int gemm_h_round(int bt);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_tn);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nn);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nt);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_tt);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_tn_bf16);
E5MA_F8_LAYOUT_DECL(launch_gemm_h_nn_bf16);
hipError_t launch_gemm_generic(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                               long long ldb, int m, int n, int k, const dev::Epilogue &e, hipStream_t s);

}  // namespace e5ma
