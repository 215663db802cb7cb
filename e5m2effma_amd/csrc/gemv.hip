// gemv.hip -- the bandwidth-bound path of e5ma_gemm: transa = T, transb = N, an FP8 A and n <= 8
// columns (reference routing src/gemm_e5m2effma.cu:100-102, kernel src/gemv_e5m2effma.cuh:27-79).
//
// D[i, j] = epilogue(sum_k A[k + i*lda] * B[k + j*ldb]).  Each wave64 owns R consecutive rows of
// op(A); lane l reads 16-byte chunks l, l + 64, ... of each row (dwordx4, fully coalesced: a wave
// reads 1 KiB contiguous per row and pass), decodes them with the packed FP8 -> FP32 converts, and
// FMAs them against the matching x values of every column.  The 64 partial sums of each output are
// combined by a butterfly over the wave; lane r*n + j then runs the epilogue of output (row r, j).
// No matrix cores: every weight byte is read once from HBM and used for n FMAs.
#include "e5ma_host.hpp"

namespace e5ma {
namespace {

using namespace dev;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// 16 FP8 codes (4 dwords) -> 16 exact FP32 values, with the hardware packed converts.  OCP decoding:
// finite codes exact (subnormals included), E5M2 Inf / NaN and E4M3 NaN codes become Inf / NaN.
template <int T> __device__ __forceinline__ void decode16(const uint32_t w[4], float v[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (T == E5MA_E5M2) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w[q], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w[q], true);
      v[4 * q] = lo[0]; v[4 * q + 1] = lo[1]; v[4 * q + 2] = hi[0]; v[4 * q + 3] = hi[1];
    } else {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], true);
      v[4 * q] = lo[0]; v[4 * q + 1] = lo[1]; v[4 * q + 2] = hi[0]; v[4 * q + 3] = hi[1];
    }
  }
}

// x values k0 .. k0 + 15 of column j as FP32 (exact decode; FP8 scale_inv is applied in the epilogue)
template <int T> __device__ __forceinline__ void load_x16(const uint8_t *B, long long ldb, int j, int k0, float v[16]) {
  const uint8_t *p = B + ((long long)j * ldb + k0) * elem_bytes(T);
  if constexpr (is_fp8(T)) {
    const uint4 q = *(const uint4 *)p;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    decode16<T>(w, v);
  } else if constexpr (T == E5MA_BF16) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint4 q = ((const uint4 *)p)[h];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * h + 2 * e] = u2f(w[e] << 16);
        v[8 * h + 2 * e + 1] = u2f(w[e] & 0xFFFF0000u);
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float4 q = ((const float4 *)p)[h];
      v[4 * h] = q.x; v[4 * h + 1] = q.y; v[4 * h + 2] = q.z; v[4 * h + 3] = q.w;
    }
  }
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o; o >>= 1) x = x + __shfl_xor(x, o, 64);
  return x;
}

template <int AT, int BT, int NB, int R, int U>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t *__restrict__ A, long long lda,
                                                        const uint8_t *__restrict__ B, long long ldb, int m, int k,
                                                        Epilogue e) {
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  const int nch = k >> 4;  // 16-byte chunks per row
  float acc[R][NB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = 0.f;
  const uint8_t *arow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) arow[r] = A + (long long)min(row0 + r, m - 1) * lda;  // rows past m: never stored

  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    uint32_t wa[U][R][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (c < nch) {
          const uint4 q = *(const uint4 *)(arow[r] + 16 * c);
          wa[u][r][0] = q.x; wa[u][r][1] = q.y; wa[u][r][2] = q.z; wa[u][r][3] = q.w;
        } else {
          wa[u][r][0] = wa[u][r][1] = wa[u][r][2] = wa[u][r][3] = 0u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c >= nch) break;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        float xv[16];
        load_x16<BT>(B, ldb, j, 16 * c, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float av[16];
          decode16<AT>(wa[u][r], av);
#pragma unroll
          for (int t = 0; t < 16; ++t) acc[r][j] = __builtin_fmaf(av[t], xv[t], acc[r][j]);
        }
      }
    }
  }

  const EpiState st = epi_begin(e);
  float mine = 0.f;
  int my_r = -1, my_j = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float s = wave_sum(acc[r][j]);
      if (lane == r * NB + j) {
        mine = s;
        my_r = r;
        my_j = j;
      }
    }
  float mx = 0.f;
  if (my_r >= 0 && row0 + my_r < m) {
    const int i = row0 + my_r;
    const float v = epi_value(e, st, i, my_j, mine);
    store_any(e.d_dtype, e.d, (size_t)my_j * e.ldd + i, v, st.qscale);
    mx = amax_fold(0.f, v);
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int AT, int BT, int NB>
hipError_t gemv_n(const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k, const Epilogue &e,
                  hipStream_t s) {
  constexpr int R = NB <= 2 ? 4 : 2;
  constexpr int U = NB <= 2 ? 4 : 2;
  const int rows_per_block = kWaves * R;
  const int grid = (m + rows_per_block - 1) / rows_per_block;
  gemv_kernel<AT, BT, NB, R, U><<<grid, kThreads, 0, s>>>(A, lda, B, ldb, m, k, e);
  return hipGetLastError();
}

template <int AT, int BT>
hipError_t gemv_b(int n, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k,
                  const Epilogue &e, hipStream_t s) {
  switch (n) {
    case 1: return gemv_n<AT, BT, 1>(A, lda, B, ldb, m, k, e, s);
    case 2: return gemv_n<AT, BT, 2>(A, lda, B, ldb, m, k, e, s);
    case 3: return gemv_n<AT, BT, 3>(A, lda, B, ldb, m, k, e, s);
    case 4: return gemv_n<AT, BT, 4>(A, lda, B, ldb, m, k, e, s);
    case 5: return gemv_n<AT, BT, 5>(A, lda, B, ldb, m, k, e, s);
    case 6: return gemv_n<AT, BT, 6>(A, lda, B, ldb, m, k, e, s);
    case 7: return gemv_n<AT, BT, 7>(A, lda, B, ldb, m, k, e, s);
    default: return gemv_n<AT, BT, 8>(A, lda, B, ldb, m, k, e, s);
  }
}

template <int AT>
hipError_t gemv_a(int bt, int n, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k,
                  const Epilogue &e, hipStream_t s) {
  switch (bt) {
    case E5MA_E5M2: return gemv_b<AT, E5MA_E5M2>(n, A, lda, B, ldb, m, k, e, s);
    case E5MA_E4M3: return gemv_b<AT, E5MA_E4M3>(n, A, lda, B, ldb, m, k, e, s);
    case E5MA_BF16: return gemv_b<AT, E5MA_BF16>(n, A, lda, B, ldb, m, k, e, s);
    default: return gemv_b<AT, E5MA_FP32>(n, A, lda, B, ldb, m, k, e, s);
  }
}

}  // namespace

hipError_t launch_gemv(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                       int k, const Epilogue &e, const DeviceInfo &, hipStream_t s) {
  if (at == E5MA_E5M2) return gemv_a<E5MA_E5M2>(bt, n, A, lda, B, ldb, m, k, e, s);
  return gemv_a<E5MA_E4M3>(bt, n, A, lda, B, ldb, m, k, e, s);
}

}  // namespace e5ma
