// gemv.hip -- the bandwidth-bound path of e5ma_gemm: transa = T, transb = N, an FP8 A and n <= 8
// columns (reference routing src/gemm_e5m2effma.cu:100-102, kernel src/gemv_e5m2effma.cuh:27-79).
//
// D[i, j] = epilogue(sum_k A[k + i*lda] * B[k + j*ldb]).  Each wave64 owns R consecutive rows of
// op(A); lane l reads 16-byte chunks l, l + 64, ... of each row (dwordx4, fully coalesced: a wave
// reads 1 KiB contiguous per row and pass), decodes them with the packed FP8 -> FP32 converts, and
// FMAs them against the matching x values of every column.  The 64 partial sums of each output are
// combined by a butterfly over the wave; lane r*n + j then runs the epilogue of output (row r, j).
// Every weight byte is read once from HBM.  At n = 1 (and for FP32 x) the products run on the VALU;
// at n = 2 .. 8 with a BF16 or FP8 x, gemv_mfma_kernel reduces 16 rows per block on the BF16 matrix
// cores, both operands staged through LDS.
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


// Epilogue operands of the one output lane `lane` finishes (row r = lane / NB, column j = lane % NB),
// fetched when the kernel starts: loaded after the reduction they would add a full memory latency to
// the end of every wave.  finish() applies the epilogue in the documented order (as epi_value does).
template <int NB> struct GemvOut {
  int r, j;
  float s, bias, c;
  __device__ __forceinline__ void fetch(const Epilogue &e, const EpiState &st, int row0, int m, int R, int lane) {
    r = lane / NB;
    j = lane - r * NB;
    const int i = min(row0 + r, m - 1);
    s = epi_scale(e, st, i, j);
    bias = e.bias ? load_any(e.bias_dtype, e.bias, (size_t)i, 1.f) : 0.f;
    c = e.beta != 0.f ? load_any(e.c_dtype, e.c, (size_t)j * e.ldc + i, st.csinv) : 0.f;
    if (r >= R) r = -1;
  }
  __device__ __forceinline__ float finish(const Epilogue &e, float acc) const {
    float v = acc * s;
    if (e.bias) v = v + bias;
    if (e.beta != 0.f) v = __builtin_fmaf(e.beta, c, v);
    return v;
  }
};

template <int AT, int BT, int NB, int R, int U>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t *__restrict__ A, long long lda,
                                                        const uint8_t *__restrict__ B, long long ldb, int m, int k,
                                                        Epilogue e) {
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  const int nch = k >> 4;  // 16-byte chunks per row
  const EpiState st = epi_begin(e);
  GemvOut<NB> out;
  out.fetch(e, st, row0, m, R, lane);
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

  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float sum = wave_sum(acc[r][j]);
      if (lane == r * NB + j) mine = sum;
    }
  float mx = 0.f;
  if (out.r >= 0 && row0 + out.r < m) {
    const int i = row0 + out.r;
    const float v = out.finish(e, mine);
    store_any(e.d_dtype, e.d, (size_t)out.j * e.ldd + i, v, st.qscale);
    mx = amax_fold(0.f, v);
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}


// ---- dot-product kernel for x in BF16, E5M2 or E4M3 --------------------------------------------
// Launch shape (rows per wave R, chunks per lane and batch U) for n <= 2 and for wider x.
#ifndef E5MA_GEMV_R_NARROW
#define E5MA_GEMV_R_NARROW 2
#endif
#ifndef E5MA_GEMV_U_NARROW
#define E5MA_GEMV_U_NARROW 4
#endif
#ifndef E5MA_GEMV_R_WIDE
#define E5MA_GEMV_R_WIDE 2
#endif
#ifndef E5MA_GEMV_U_WIDE
#define E5MA_GEMV_U_WIDE 4
#endif
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 4 FP8 codes of a dword -> 2 packed BF16 pairs, exactly (every finite FP8 value is a BF16 value)
template <int T> __device__ __forceinline__ void fp8x4_to_bf16(uint32_t w, bf16x2 &lo, bf16x2 &hi) {
  if constexpr (T == E5MA_E5M2) {
    lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8((int)w, 1.0f, false);
    hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8((int)w, 1.0f, true);
  } else {
    lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false);
    hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true);
  }
}

// x values 16c .. 16c + 15 of column j as 8 BF16 pairs (raw for BF16 x, converted for FP8 x)
template <int BT> struct XChunk {
  static constexpr int kDw = is_fp8(BT) ? 4 : 8;  // dwords loaded per chunk
  uint32_t w[kDw];
  __device__ __forceinline__ void load(const uint8_t *B, long long ldb, int j, int c) {
    const u32x4 *p = (const u32x4 *)(B + ((long long)j * ldb + 16 * c) * elem_bytes(BT));
#pragma unroll
    for (int h = 0; h < kDw / 4; ++h) {
      const u32x4 q = p[h];
      w[4 * h] = q[0]; w[4 * h + 1] = q[1]; w[4 * h + 2] = q[2]; w[4 * h + 3] = q[3];
    }
  }
  __device__ __forceinline__ void pairs(bf16x2 xp[8], bool valid) const {
    if constexpr (is_fp8(BT)) {
#pragma unroll
      for (int d = 0; d < 4; ++d) fp8x4_to_bf16<BT>(valid ? w[d] : 0u, xp[2 * d], xp[2 * d + 1]);
    } else {
#pragma unroll
      for (int d = 0; d < 8; ++d) xp[d] = __builtin_bit_cast(bf16x2, valid ? w[d] : 0u);
    }
  }
};

// Each wave64 owns R rows.  A batch issues every weight load of U chunks per lane (non-temporal
// dwordx4, branch-free: chunk indices are clamped and chunks past the row end are zeroed after the
// load), then the x chunks; the compute follows the loads as they land (they complete in order).  Per
// 16 weights and row: 8 v_cvt_scalef32_pk_bf16_{bf8,fp8} and 8 v_dot2_f32_bf16 (products exact,
// FP32 accumulation), with x shared by the R rows.
template <int AT, int BT, int NB, int R, int U>
// (A and B are not __restrict__: loads through restrict pointers may be moved across the fence
// that keeps the x loads ahead of the weight loads.)
__global__ __launch_bounds__(kThreads) void gemv_dot_kernel(const uint8_t *A, long long lda, const uint8_t *B,
                                                            long long ldb, int m, int k, Epilogue e) {
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  const int nch = k >> 4;
  const EpiState st = epi_begin(e);
  GemvOut<NB> out;
  out.fetch(e, st, row0, m, R, lane);
  const uint8_t *arow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) arow[r] = A + (long long)min(row0 + r, m - 1) * lda;  // rows past m: never stored
  float acc[R][NB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = 0.f;

  // x up front (NB <= 2): its loads are then older than the weight loads, so the first chunk's
  // products can start as soon as its weights land (vector-memory loads complete in order)
  constexpr bool kXUp = NB <= 2;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    XChunk<BT> xup[kXUp ? U : 1][kXUp ? NB : 1];
    if constexpr (kXUp) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < NB; ++j) xup[u][j].load(B, ldb, j, min(c0 + 64 * u, nch - 1));
      asm volatile("" ::: "memory");
    }
    u32x4 wa[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + 64 * u, nch - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) wa[u][r] = __builtin_nontemporal_load((const u32x4 *)(arow[r] + 16 * c));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      const bool valid = c < nch;
      const int cc = valid ? c : nch - 1;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        XChunk<BT> xc;
        if constexpr (kXUp) xc = xup[u][j];
        else xc.load(B, ldb, j, cc);
        bf16x2 xp[8];
        xc.pairs(xp, valid);
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            bf16x2 lo, hi;
            fp8x4_to_bf16<AT>(valid ? wa[u][r][d] : 0u, lo, hi);
            acc[r][j] = __builtin_amdgcn_fdot2_f32_bf16(lo, xp[2 * d], acc[r][j], false);
            acc[r][j] = __builtin_amdgcn_fdot2_f32_bf16(hi, xp[2 * d + 1], acc[r][j], false);
          }
        }
      }
    }
  }

  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float sum = wave_sum(acc[r][j]);
      if (lane == r * NB + j) mine = sum;
    }
  float mx = 0.f;
  if (out.r >= 0 && row0 + out.r < m) {
    const int i = row0 + out.r;
    const float v = out.finish(e, mine);
    store_any(e.d_dtype, e.d, (size_t)out.j * e.ldd + i, v, st.qscale);
    mx = amax_fold(0.f, v);
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

// ---- x staged in LDS by direct-to-LDS loads (BF16 / FP16 / FP8 x of at most kXLds bytes) ----------
constexpr int kXLds = 131072;
#ifndef E5MA_GEMV_RX
#define E5MA_GEMV_RX 2  // rows per wave
#endif
#ifndef E5MA_GEMV_UX
#define E5MA_GEMV_UX 4  // 16-byte chunks per lane and row in flight
#endif
// n > 2 (measured on 8192^2: n = 4 best with 2 rows x 2 chunks, 16.5 us; n = 8 with 4 rows x 2 chunks,
// 24.6 us, where the FP32 FMA kernel took 24.1 / 34.1 us; 2 rows x 4 chunks spill at n = 8)
template <int NB> constexpr int kGemvRxWide = NB <= 4 ? 2 : 4;
constexpr int kGemvUxWide = 2;
typedef __attribute__((address_space(3))) void lds_void_t;

// one direct-to-LDS load: 16 bytes per lane from src to lds + 16 * lane (lds wave-uniform); inline asm,
// so that it is ordered with the barrier asm below and not counted by the compiler's wait-count pass.
// It sets m0 itself; the compiler emits no other m0 use in this file (checked in the generated code).
__device__ __forceinline__ void gemv_load_lds16(const uint8_t *src, const uint8_t *lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "memory", "m0");
}

// x values 16c .. 16c + 15 of column j from the LDS copy (column j at xs + j * k * bytes(x))
template <int BT> __device__ __forceinline__ void xlds_pairs(const uint8_t *xs, int k, int j, int c, bool valid,
                                                            bf16x2 xp[8]) {
  const uint8_t *p = xs + ((long long)j * k + 16 * c) * elem_bytes(BT);
  XChunk<BT> xc;
#pragma unroll
  for (int h = 0; h < XChunk<BT>::kDw / 4; ++h) {
    const uint4 q = ((const uint4 *)p)[h];
    xc.w[4 * h] = q.x; xc.w[4 * h + 1] = q.y; xc.w[4 * h + 2] = q.z; xc.w[4 * h + 3] = q.w;
  }
  xc.pairs(xp, valid);
}

// As gemv_dot_kernel, but the block first copies x into LDS with direct-to-LDS loads (issued before
// the weight loads, so they complete first), then waits only for those, so x never occupies the
// vector-memory pipe again and the weights stream alone.
// 512-thread blocks, 2 rows and 4 chunks per lane and batch (measured best of 1 / 2 / 4 rows, 4 / 8
// chunks and 256 / 512 / 1024-thread blocks on the 8192 x 8192 batch-1 and -2 shapes: 512 threads halve
// the x copies of 256 (13.1 vs 13.7 us at n = 1); 8 chunks need 140 VGPRs, too many for the grid's
// 4 waves per SIMD)
#ifndef E5MA_GEMV_XTHREADS
#define E5MA_GEMV_XTHREADS 512
#endif
constexpr int kXThreads = E5MA_GEMV_XTHREADS, kXWaves = kXThreads / 64;
template <int AT, int BT, int NB, int R, int U>
__global__ __launch_bounds__(kXThreads) void gemv_xlds_kernel(const uint8_t *A, long long lda, const uint8_t *B,
                                                             long long ldb, int m, int k, Epilogue e) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t xs[];  // x, rounded up to whole KiB
  __shared__ float red[kXWaves];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (blockIdx.x * kXWaves + wave) * R;
  const int nch = k >> 4;
  const EpiState st = epi_begin(e);
  GemvOut<NB> out;
  out.fetch(e, st, row0, m, R, lane);
  const int colbytes = k * elem_bytes(BT), xtotal = colbytes * NB;
  // x: 1 KiB per wave and step into the dynamic LDS of round_up(xtotal, 1 KiB); source offsets past
  // the end are clamped (the bytes they land on are never read)
  constexpr int kSteps = kXLds / (1024 * kXWaves);
#pragma unroll
  for (int q = 0; q < kSteps; ++q) {
    const int blk = q * kXWaves + wave;
    if (blk * 1024 < xtotal) {  // wave-uniform
      const int o = min(blk * 1024 + 16 * lane, xtotal - 16);
      const int j = o / colbytes, w = o - j * colbytes;
      gemv_load_lds16(B + (long long)j * ldb * elem_bytes(BT) + w, xs + blk * 1024);
    }
  }
  const uint8_t *arow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) arow[r] = A + (long long)min(row0 + r, m - 1) * lda;
  float acc[R][NB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = 0.f;

  bool first = true;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    u32x4 wa[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + 64 * u, nch - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) wa[u][r] = __builtin_nontemporal_load((const u32x4 *)(arow[r] + 16 * c));
    }
    if (first) {
      // x landed (the U * R weight loads just issued may stay in flight), visible to the whole block
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(U * R) : "memory");
      first = false;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      const bool valid = c < nch;
      const int cc = valid ? c : nch - 1;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        bf16x2 xp[8];
        xlds_pairs<BT>(xs, k, j, cc, valid, xp);
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            bf16x2 lo, hi;
            fp8x4_to_bf16<AT>(valid ? wa[u][r][d] : 0u, lo, hi);
            acc[r][j] = __builtin_amdgcn_fdot2_f32_bf16(lo, xp[2 * d], acc[r][j], false);
            acc[r][j] = __builtin_amdgcn_fdot2_f32_bf16(hi, xp[2 * d + 1], acc[r][j], false);
          }
        }
      }
    }
  }
  if (first) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // no chunk: still drain and sync

  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float sum = wave_sum(acc[r][j]);
      if (lane == r * NB + j) mine = sum;
    }
  float mx = 0.f;
  if (out.r >= 0 && row0 + out.r < m) {
    const int i = row0 + out.r;
    const float v = out.finish(e, mine);
    store_any(e.d_dtype, e.d, (size_t)out.j * e.ldd + i, v, st.qscale);
    mx = amax_fold(0.f, v);
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

// ---- matrix-core kernel for 2 <= n <= 8 with BF16 or FP8 x ----------------------------------------
// A block owns 16 rows and reduces them over all of k on v_mfma_f32_16x16x32_bf16: operand A is the 16
// rows of weights widened exactly to BF16, operand B is x widened the same way (BF16 x as is), with
// columns n .. 15 of the 16-column operand zero.  Lane l (row / column r = l & 15, k-group g = l >> 4)
// takes chunks t = g + 4u (u < U) of each batch of 4U 16-byte chunks per row; MFMA (u, h) takes k
// 16 t + 8 h .. + 7 for A from row r and for B from column r of x at the same k.  Any assignment of k to
// the 32 slots of one MFMA is a valid reduction order as long as A and B use the same one, and they do.
// Products are exact and accumulate in FP32, so the result meets the same bound as the dot kernels.
// Both operands of a batch reach the wave through its own LDS slot, filled by direct-to-LDS loads one
// batch ahead: the weights as whole 128-byte lines of 16 / U rows per 1 KiB load, x as whole columns of
// the batch's k range.  Loaded straight into registers in the MFMA layout, every weight instruction read
// 64-byte halves of 16 rows and every x instruction 16 bytes from each of up to 32 lines (8 columns
// 16 KiB apart, 4 k-groups): about 300 line requests per batch against about 60 now, and the time was
// flat in n.  The W waves of a block take every W-th batch; their 16 x 16 partial results are summed in
// wave order through LDS (deterministic), then 16 n threads run the epilogue.
// Measured on 8192 x 8192 E5M2 x BF16 (us; dot kernels / earlier register-loaded MFMA kernel -> this one,
// U = 2, 4 waves): n = 1 11.9 -> 12.4 (so n = 1 stays on the dot kernel), n = 2 13.0 -> 12.4, n = 4
// 16.3 -> 12.7, n = 8 21.1 -> 13.0; U = 4 14.7 and 2 waves per block 15.7 at n = 8.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#ifndef E5MA_GEMV_MFMA_MIN_N
#define E5MA_GEMV_MFMA_MIN_N 2  // smallest n on this kernel
#endif
#ifndef E5MA_GEMV_MFMA_U
#define E5MA_GEMV_MFMA_U 2  // 16-byte chunks per lane and batch
#endif
#ifndef E5MA_GEMV_MFMA_WAVES
#define E5MA_GEMV_MFMA_WAVES 4
#endif
constexpr int kMWaves = E5MA_GEMV_MFMA_WAVES, kMThreads = 64 * kMWaves;

// One batch of gemv_mfma_kernel: U chunks per lane (c = cl + 4 u) loaded, widened and multiplied.  FULL
// batches (every chunk inside the row: the wave-uniform cw + 4 U <= nch) take unclamped addresses and no
// masks; the last, partial batch clamps its addresses and zeroes out-of-range chunks as whole 32-bit words
// (weights and x both, so that no x value past the row end meets a weight).
// x of one batch in LDS: for each of the 8 columns the batch's 64 U values of k (kColBytes bytes) as 16-byte
// chunks, chunk t of column j at position t ^ (j & kSwz).  The 16 lanes that read one MFMA's B fragments
// (columns r = 0..15 at one chunk) then meet 16 distinct bank groups (lanes r and r + 8 read the same
// address).  Filled by direct-to-LDS loads of 1 KiB, each a whole number of columns: lane s fetches
// the chunk its LDS position holds, so the lanes of one column read its bytes contiguously.
template <int BT, int U> struct XSlice {
  static constexpr int kColBytes = 64 * U * elem_bytes(BT);
  static constexpr int kChunks = kColBytes / 16;         // 16-byte chunks per column
  static constexpr int kSwz = kChunks - 1 < 15 ? kChunks - 1 : 15;
  static constexpr int kBytes = 8 * kColBytes;
  static constexpr int kLoads = kBytes / 1024;          // 1 KiB loads per slice of 8 columns
  static constexpr int kColsPerLoad = 1024 / kColBytes;
  static_assert(kBytes % 1024 == 0 && kChunks <= 64, "whole columns per 1 KiB load");
  // loads that cover columns 0 .. nb - 1 (the slots of the others are never read unmasked)
  static constexpr int loads_for(int nb) { return (nb + kColsPerLoad - 1) / kColsPerLoad; }
};

// Issues the direct-to-LDS loads of the x slice for chunks c0 .. c0 + 4U - 1 of the weight row (k = 16 c0 ..)
// into xs; columns past n repeat column n - 1 and chunks past the row end repeat its last chunk (read
// but never multiplied: their weights and x are masked)
template <int BT, int U, int NB>
__device__ __forceinline__ void xslice_issue(uint8_t *xs, const uint8_t *B, long long ldb, int n, int c0, int nch,
                                             int lane) {
  using X = XSlice<BT, U>;
  constexpr int kColsPerLoad = X::kColsPerLoad;
#pragma unroll
  for (int q = 0; q < X::loads_for(NB); ++q) {
    const int j = q * kColsPerLoad + lane / X::kChunks, pos = lane % X::kChunks;
    const int t = pos ^ (j & X::kSwz);                                   // chunk of column j this lane fetches
    const long long kk = min(16LL * c0 + (long long)t * (16 / elem_bytes(BT)), 16LL * nch - 16 / elem_bytes(BT));
    const uint8_t *src = B + ((long long)min(j, n - 1) * ldb + kk) * elem_bytes(BT);
    gemv_load_lds16(src, xs + 1024 * q);
  }
}

// B fragment of MFMA (u, h) for this lane (column r, k-group g) from the x slice: x values of k
// 16 (g + 4u) + 8h .. + 7 of column r & 7 as 4 dwords of BF16 pairs
template <int BT, int U>
__device__ __forceinline__ u32x4 xslice_frag(const uint8_t *xs, int r, int g, int u, int h) {
  using X = XSlice<BT, U>;
  const int j = r & 7;
  if constexpr (is_fp8(BT)) {
    const int t = g + 4 * u;  // 16-byte chunk (16 codes), half h
    const uint2 w = *(const uint2 *)(xs + j * X::kColBytes + 16 * (t ^ (j & X::kSwz)) + 8 * h);
    bf16x2 p0, p1, p2, p3;
    fp8x4_to_bf16<BT>(w.x, p0, p1);
    fp8x4_to_bf16<BT>(w.y, p2, p3);
    return u32x4{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1), __builtin_bit_cast(uint32_t, p2),
                 __builtin_bit_cast(uint32_t, p3)};
  } else {
    const int t = 2 * (g + 4 * u) + h;  // 16-byte chunk (8 BF16 values)
    return *(const u32x4 *)(xs + j * X::kColBytes + 16 * (t ^ (j & X::kSwz)));
  }
}

// The weights of one batch in LDS: 16 rows of 4 U chunks of 16 bytes (the batch's 64 U bytes of k), chunk t
// of row r at position t ^ (r & kSwz), so that the 16 lanes reading one MFMA's A fragments (rows 0..15
// at one chunk) meet distinct bank groups.  Filled by 1 KiB direct-to-LDS loads of 16 / U rows each:
// lane s fetches the chunk its position holds, so the lanes of one row read its bytes contiguously
// (whole 128-byte lines).
template <int U> struct WSlice {
  static constexpr int kChunks = 4 * U;                 // chunks per row and batch
  static constexpr int kSwz = kChunks - 1 < 15 ? kChunks - 1 : 15;
  static constexpr int kBytes = 16 * 16 * kChunks;
  static constexpr int kLoads = kBytes / 1024;
  static constexpr int kRowsPerLoad = 64 / kChunks;
  static_assert(kBytes % 1024 == 0 && 64 % kChunks == 0, "whole rows per 1 KiB load");
};

// Issues the weight loads of the batch at chunks c0 .. c0 + 4U - 1 of rows i0 .. i0 + 15 (rows past m
// repeat row m - 1, chunks past the row end its last chunk: read, never multiplied)
template <int U>
__device__ __forceinline__ void wslice_issue(uint8_t *ws, const uint8_t *A, long long lda, int i0, int m, int c0,
                                             int nch, int lane) {
  using W = WSlice<U>;
#pragma unroll
  for (int q = 0; q < W::kLoads; ++q) {
    const int r = q * W::kRowsPerLoad + lane / W::kChunks, pos = lane % W::kChunks;
    const int t = pos ^ (r & W::kSwz);
    const uint8_t *src = A + (long long)min(i0 + r, m - 1) * lda + 16LL * min(c0 + t, nch - 1);
    gemv_load_lds16(src, ws + 1024 * q);
  }
}

// One batch's products from the two slices: A fragment (u, h) of lane (row r, group g) is half h of
// chunk g + 4u of row r, widened exactly to BF16; chunks past the row end (FULL false) are zeroed as
// whole words in the weights and x both
template <int AT, int BT, int U, bool FULL>
__device__ __forceinline__ void gemv_mfma_compute(const uint8_t *ws, const uint8_t *xs, int r, int g, bool xlane,
                                                  int cl, int nch, f32x4 &acc) {
  using W = WSlice<U>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t keep = FULL || cl + 4 * u < nch ? ~0u : 0u, xkeep = xlane ? keep : 0u;
    const int t = g + 4 * u;
    const u32x4 wa = *(const u32x4 *)(ws + r * (16 * W::kChunks) + 16 * (t ^ (r & W::kSwz)));
    uint32_t aw[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      bf16x2 lo, hi;
      fp8x4_to_bf16<AT>(wa[d] & keep, lo, hi);
      aw[2 * d] = __builtin_bit_cast(uint32_t, lo);
      aw[2 * d + 1] = __builtin_bit_cast(uint32_t, hi);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 xb = xslice_frag<BT, U>(xs, r, g, u, h);
      const u32x4 av = {aw[4 * h], aw[4 * h + 1], aw[4 * h + 2], aw[4 * h + 3]};
      const u32x4 bv = {xb[0] & xkeep, xb[1] & xkeep, xb[2] & xkeep, xb[3] & xkeep};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), acc,
                                                    0, 0, 0);
    }
  }
}

template <int AT, int BT, int NB, int U>
__global__ __launch_bounds__(kMThreads) void gemv_mfma_kernel(const uint8_t *A, long long lda, const uint8_t *B,
                                                             long long ldb, int m, int k, Epilogue e) {
  using X = XSlice<BT, U>;
  using W = WSlice<U>;
  constexpr int kSlot = W::kBytes + X::kBytes;  // one batch of one wave in LDS: weights, then x
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kMWaves][2][kSlot];
  __shared__ float part[kMWaves][16][17];
  __shared__ float red[kMWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int i0 = blockIdx.x * 16;
  const int nch = k >> 4;
  const EpiState st = epi_begin(e);
  GemvOut<NB> out;
  out.fetch(e, st, i0, m, 16, tid);
  const bool xlane = r < NB;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // Batches b = 0, 1, ... of this wave at chunks cw0 + b kStep (the last may be partial), both operands
  // staged in this wave's two LDS slots by direct-to-LDS loads one batch ahead of the products.  Those
  // loads are inline asm, invisible to the compiler, and no other vector-memory load is in the loop:
  // the explicit wait before each batch (everything but the next batch's loads landed) is the only one.
  constexpr int kStep = kMWaves * 4 * U, kPerBatch = W::kLoads + X::loads_for(NB);
  const int cw0 = wave * 4 * U;
  const int nb = cw0 < nch ? (nch - 1 - cw0) / kStep + 1 : 0;
  if (nb > 0) {
    wslice_issue<U>(lds[wave][0], A, lda, i0, m, cw0, nch, lane);
    xslice_issue<BT, U, NB>(lds[wave][0] + W::kBytes, B, ldb, NB, cw0, nch, lane);
  }
  for (int b = 0; b < nb; ++b) {
    const int cw = cw0 + b * kStep;
    uint8_t *slot = lds[wave][b & 1];
    if (b + 1 < nb) {
      // the other slot was last read by batch b - 1, whose products are done
      uint8_t *next = lds[wave][(b + 1) & 1];
      wslice_issue<U>(next, A, lda, i0, m, cw + kStep, nch, lane);
      xslice_issue<BT, U, NB>(next + W::kBytes, B, ldb, NB, cw + kStep, nch, lane);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPerBatch) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    if (cw + 4 * U <= nch) gemv_mfma_compute<AT, BT, U, true>(slot, slot + W::kBytes, r, g, xlane, cw + g, nch, acc);
    else gemv_mfma_compute<AT, BT, U, false>(slot, slot + W::kBytes, r, g, xlane, cw + g, nch, acc);
  }
  // lane l holds outputs (row 4 g + q, column r) of its wave's partial result
#pragma unroll
  for (int q = 0; q < 4; ++q) part[wave][4 * g + q][r] = acc[q];
  __syncthreads();
  float mx = 0.f;
  if (out.r >= 0 && i0 + out.r < m) {
    float sum = part[0][out.r][out.j];
#pragma unroll
    for (int w = 1; w < kMWaves; ++w) sum += part[w][out.r][out.j];
    const float v = out.finish(e, sum);
    store_any(e.d_dtype, e.d, (size_t)out.j * e.ldd + i0 + out.r, v, st.qscale);
    mx = amax_fold(0.f, v);
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int AT, int BT, int NB>
hipError_t gemv_n(const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k, const Epilogue &e,
                  const Tuning &tu, hipStream_t s) {
  if constexpr (BT != E5MA_FP32 && NB >= E5MA_GEMV_MFMA_MIN_N) {
    gemv_mfma_kernel<AT, BT, NB, E5MA_GEMV_MFMA_U><<<(m + 15) / 16, kMThreads, 0, s>>>(A, lda, B, ldb, m, k, e);
    return hipGetLastError();
  }
  if constexpr (BT != E5MA_FP32) {
    const long long xbytes = (long long)k * NB * elem_bytes(BT);
    if (xbytes <= kXLds) {
      const size_t lds = (size_t)((xbytes + 1023) / 1024 * 1024);
      if constexpr (NB == 1) {
        // rows per wave from the tuned table (the tuner's candidates; every one sums a row in the same order)
        if (tu.gemv_rows == 1) {
          gemv_xlds_kernel<AT, BT, 1, 1, 8><<<(m + kXWaves - 1) / kXWaves, kXThreads, lds, s>>>(A, lda, B, ldb, m, k, e);
          return hipGetLastError();
        }
        if (tu.gemv_rows == 4) {
          gemv_xlds_kernel<AT, BT, 1, 4, 2><<<(m + 4 * kXWaves - 1) / (4 * kXWaves), kXThreads, lds, s>>>(A, lda, B, ldb,
                                                                                                           m, k, e);
          return hipGetLastError();
        }
      }
      constexpr int RX = NB <= 2 ? E5MA_GEMV_RX : kGemvRxWide<NB>, UX = NB <= 2 ? E5MA_GEMV_UX : kGemvUxWide;
      const int gx = (m + kXWaves * RX - 1) / (kXWaves * RX);
      gemv_xlds_kernel<AT, BT, NB, RX, UX><<<gx, kXThreads, lds, s>>>(A, lda, B, ldb, m, k, e);
      return hipGetLastError();
    }
    if constexpr (NB <= 2) {
      constexpr int R = E5MA_GEMV_R_NARROW, U = E5MA_GEMV_U_NARROW;
      const int grid = (m + kWaves * R - 1) / (kWaves * R);
      gemv_dot_kernel<AT, BT, NB, R, U><<<grid, kThreads, 0, s>>>(A, lda, B, ldb, m, k, e);
      return hipGetLastError();
    }
  }
  // FP32 x is not a BF16 value; a wide x that does not fit LDS: the FP32 FMA kernel
  constexpr int R = NB <= 2 ? 4 : 2;
  constexpr int U = NB <= 2 ? 4 : 2;
  const int rows_per_block = kWaves * R;
  const int grid = (m + rows_per_block - 1) / rows_per_block;
  gemv_kernel<AT, BT, NB, R, U><<<grid, kThreads, 0, s>>>(A, lda, B, ldb, m, k, e);
  return hipGetLastError();
}

template <int AT, int BT>
hipError_t gemv_b(int n, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k,
                  const Epilogue &e, const Tuning &tu, hipStream_t s) {
  switch (n) {
    case 1: return gemv_n<AT, BT, 1>(A, lda, B, ldb, m, k, e, tu, s);
    case 2: return gemv_n<AT, BT, 2>(A, lda, B, ldb, m, k, e, tu, s);
    case 3: return gemv_n<AT, BT, 3>(A, lda, B, ldb, m, k, e, tu, s);
    case 4: return gemv_n<AT, BT, 4>(A, lda, B, ldb, m, k, e, tu, s);
    case 5: return gemv_n<AT, BT, 5>(A, lda, B, ldb, m, k, e, tu, s);
    case 6: return gemv_n<AT, BT, 6>(A, lda, B, ldb, m, k, e, tu, s);
    case 7: return gemv_n<AT, BT, 7>(A, lda, B, ldb, m, k, e, tu, s);
    default: return gemv_n<AT, BT, 8>(A, lda, B, ldb, m, k, e, tu, s);
  }
}

template <int AT>
hipError_t gemv_a(int bt, int n, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int k,
                  const Epilogue &e, const Tuning &tu, hipStream_t s) {
  switch (bt) {
    case E5MA_E5M2: return gemv_b<AT, E5MA_E5M2>(n, A, lda, B, ldb, m, k, e, tu, s);
    case E5MA_E4M3: return gemv_b<AT, E5MA_E4M3>(n, A, lda, B, ldb, m, k, e, tu, s);
    case E5MA_BF16: return gemv_b<AT, E5MA_BF16>(n, A, lda, B, ldb, m, k, e, tu, s);
    default: return gemv_b<AT, E5MA_FP32>(n, A, lda, B, ldb, m, k, e, tu, s);
  }
}

}  // namespace

hipError_t launch_gemv(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                       int k, const Epilogue &e, const DeviceInfo &di, hipStream_t s) {
  if (at == E5MA_E5M2) return gemv_a<E5MA_E5M2>(bt, n, A, lda, B, ldb, m, k, e, di.tune, s);
  return gemv_a<E5MA_E4M3>(bt, n, A, lda, B, ldb, m, k, e, di.tune, s);
}

}  // namespace e5ma
