// gemm_generic.hip -- the tiled path of e5ma_gemm for every operand pairing and layout (reference
// src/gemm_e5m2effma.cuh:117-233, which computes the same product with one FFMA per MAC).
//
// Three arithmetic modes on the gfx950 matrix cores, each exact in its products:
//   F8: both operands FP8 (E5M2 / E4M3, any pairing) -> v_mfma_scale_f32_32x32x64_f8f6f4 with neutral
//       E8M0 scales (2^0); the operands stay in their 1-byte codes.
//   H:  a BF16 operand and no FP32 one -> FP8 operands upcast exactly to BF16,
//       v_mfma_f32_32x32x16_bf16.
//   S:  an FP32 operand -> everything decoded exactly to FP32, v_mfma_f32_32x32x2_f32.
// Block tile 128 x 128 (4 waves, 2 x 2, each 64 x 64 = 2 x 2 MFMA blocks of 32 x 32), K staged in
// 64-byte LDS rows (64 FP8, 32 BF16 or 16 FP32 values), two LDS buffers, one barrier per stage, the
// next stage prefetched into registers while the current one is multiplied.  The 16-byte chunks of
// each LDS row are XOR-swizzled by row so that the fragment reads of 8 consecutive rows hit 32
// distinct banks.  Operands stored K-contiguous are read with dwordx4 loads; M/N-contiguous ones
// are gathered element by element (lanes run along the contiguous dimension, so each load
// instruction of a wave still covers contiguous memory).
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {
namespace {

using namespace dev;
using namespace gemm;

constexpr int kBM = 128, kBN = 128, kThreads = 256;
constexpr int kRowBytes = 64;                    // one LDS row: 64 bytes of K
constexpr int kTileBytes = kBM * kRowBytes;      // 8 KiB per operand and stage
constexpr int kStageLd = kBM + 4;                // staged accumulators: [64 columns][kBM + 4] floats
constexpr int kSmemBytes = 64 * kStageLd * 4 > 4 * kTileBytes ? 64 * kStageLd * 4 : 4 * kTileBytes;

template <int MODE> struct ModeTraits;
template <> struct ModeTraits<kModeF8> { static constexpr int csize = 1; };
template <> struct ModeTraits<kModeH> { static constexpr int csize = 2; };
template <> struct ModeTraits<kModeS> { static constexpr int csize = 4; };

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

// One operand's share of a stage: 32 bytes of compute-type values for LDS row `row`, half `half`.
template <int MODE, int T, bool KC> struct Loader {
  static constexpr int kCs = ModeTraits<MODE>::csize;
  static constexpr int kE = 32 / kCs;  // compute values per thread and stage
  uint32_t w[8];

  // value t of the thread's range as compute-type bits (kCs bytes), from element (r, kk)
  __device__ __forceinline__ static uint32_t conv(float x) {
    if constexpr (kCs == 2) return __float_as_uint(x) >> 16;  // exact: the value is a BF16 value
    else return __float_as_uint(x);
  }

  __device__ __forceinline__ void load(const uint8_t *base, long long ld, int rows, int r, int k0, int k, int half) {
    r = min(r, rows - 1);
    const int kb = k0 + half * kE;
    if constexpr (KC) {
      const uint8_t *p = base + ((long long)r * ld + kb) * elem_bytes(T);
      // 16-value groups (k and the stage offsets are multiples of 16 values, 8 for FP32 mode)
      constexpr int kGroup = kE < 16 ? kE : 16;
#pragma unroll
      for (int g = 0; g < kE / kGroup; ++g) {
        const bool in = kb + g * kGroup < k;
        if constexpr (MODE == kModeF8) {  // 16 FP8 codes -> 4 dwords
          uint4 q = make_uint4(0, 0, 0, 0);
          if (in) q = *(const uint4 *)(p + g * 16);
          w[4 * g] = q.x; w[4 * g + 1] = q.y; w[4 * g + 2] = q.z; w[4 * g + 3] = q.w;
        } else {
          float v[16];
#pragma unroll
          for (int t = 0; t < kGroup; ++t) v[t] = 0.f;
          if (in) load_group<T, kGroup>(p + g * kGroup * elem_bytes(T), v);
#pragma unroll
          for (int t = 0; t < kGroup; t += 4 / kCs) {
            if constexpr (kCs == 2) w[(g * kGroup + t) / 2] = conv(v[t]) | (conv(v[t + 1]) << 16);
            else w[g * kGroup + t] = conv(v[t]);
          }
        }
      }
    } else {
      // element (r, kk) at base[r + kk * ld]
#pragma unroll
      for (int t = 0; t < kE; ++t) {
        const int kk = kb + t;
        uint32_t bits = 0;
        if (kk < k) {
          const long long idx = (long long)kk * ld + r;
          if constexpr (MODE == kModeF8) bits = base[idx];
          else bits = conv(operand_value<T>(base, idx));
        }
        if constexpr (kCs == 1) {
          if (t % 4 == 0) w[t / 4] = 0;
          w[t / 4] |= bits << (8 * (t % 4));
        } else if constexpr (kCs == 2) {
          if (t % 2 == 0) w[t / 2] = 0;
          w[t / 2] |= bits << (16 * (t % 2));
        } else {
          w[t] = bits;
        }
      }
    }
  }
  __device__ __forceinline__ void store(uint8_t *lds, int row, int half) const {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int chunk = swz(row, 2 * half + c);
      *(uint4 *)(lds + row * kRowBytes + chunk * 16) = make_uint4(w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]);
    }
  }
};

template <int MODE, int AT, int BT, bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads) void gemm_generic_kernel(const uint8_t *__restrict__ A, long long lda,
                                                                const uint8_t *__restrict__ B, long long ldb, int m,
                                                                int n, int k, Epilogue e) {
  // operand stages [buffer][A / B], reused after the K loop to stage half a tile of accumulators
  __shared__ __attribute__((aligned(16))) uint8_t smem[kSmemBytes];
  __shared__ float red[kThreads / 64];
  uint8_t(*lds)[2][kTileBytes] = (uint8_t(*)[2][kTileBytes])smem;
  constexpr int kCs = ModeTraits<MODE>::csize;
  constexpr int kBK = kRowBytes / kCs;  // K values per stage
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int i0 = blockIdx.y * kBM, j0 = blockIdx.x * kBN;
  // K-contiguous operands: thread -> (row t / 2, half t % 2); M/N-contiguous: (row t % 128, half t / 128)
  const int ar = AKC ? tid >> 1 : tid & 127, ah = AKC ? tid & 1 : tid >> 7;
  const int br = BKC ? tid >> 1 : tid & 127, bh = BKC ? tid & 1 : tid >> 7;
  Loader<MODE, AT, AKC> la;
  Loader<MODE, BT, BKC> lb;

  v16f acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  const int nst = (k + kBK - 1) / kBK;
  // operand rows are offset by the tile origin: A row i0 + ar, B row (column of op(B)) j0 + br
  const uint8_t *Ap = AKC ? A + (long long)i0 * lda * elem_bytes(AT) : A + (long long)i0 * elem_bytes(AT);
  const uint8_t *Bp = BKC ? B + (long long)j0 * ldb * elem_bytes(BT) : B + (long long)j0 * elem_bytes(BT);
  const int arows = m - i0, brows = n - j0;
  if (nst > 0) {
    la.load(Ap, lda, arows, ar, 0, k, ah);
    lb.load(Bp, ldb, brows, br, 0, k, bh);
    la.store(lds[0][0], ar, ah);
    lb.store(lds[0][1], br, bh);
  }
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1;
    if (s + 1 < nst) {
      la.load(Ap, lda, arows, ar, (s + 1) * kBK, k, ah);
      lb.load(Bp, ldb, brows, br, (s + 1) * kBK, k, bh);
    }
    const uint8_t *sa = lds[buf][0], *sb = lds[buf][1];
    if constexpr (MODE == kModeF8) {
      v8i fa[2], fb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int ra = wm * 64 + x * 32 + (lane & 31), rb = wn * 64 + x * 32 + (lane & 31);
        const int c0 = 2 * (lane >> 5);
        const uint4 a0 = *(const uint4 *)(sa + ra * kRowBytes + swz(ra, c0) * 16);
        const uint4 a1 = *(const uint4 *)(sa + ra * kRowBytes + swz(ra, c0 + 1) * 16);
        const uint4 b0 = *(const uint4 *)(sb + rb * kRowBytes + swz(rb, c0) * 16);
        const uint4 b1 = *(const uint4 *)(sb + rb * kRowBytes + swz(rb, c0 + 1) * 16);
        fa[x] = v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        fb[x] = v8i{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[x], fb[y], acc[x][y], kMfmaFmt<AT>,
                                                                      kMfmaFmt<BT>, 0, kNeutralScale, 0,
                                                                      kNeutralScale);
    } else if constexpr (MODE == kModeH) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {  // two K steps of 16 per stage
        v8bf fa[2], fb[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int ra = wm * 64 + x * 32 + (lane & 31), rb = wn * 64 + x * 32 + (lane & 31);
          const int c = 2 * st + (lane >> 5);
          fa[x] = __builtin_bit_cast(v8bf, *(const uint4 *)(sa + ra * kRowBytes + swz(ra, c) * 16));
          fb[x] = __builtin_bit_cast(v8bf, *(const uint4 *)(sb + rb * kRowBytes + swz(rb, c) * 16));
        }
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y) acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[x], fb[y], acc[x][y], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int st = 0; st < 8; ++st) {  // eight K steps of 2 per stage
        float fa[2], fb[2];
        const int byte = 8 * st + 4 * (lane >> 5);
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int ra = wm * 64 + x * 32 + (lane & 31), rb = wn * 64 + x * 32 + (lane & 31);
          fa[x] = *(const float *)(sa + ra * kRowBytes + swz(ra, byte >> 4) * 16 + (byte & 15));
          fb[x] = *(const float *)(sb + rb * kRowBytes + swz(rb, byte >> 4) * 16 + (byte & 15));
        }
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y) acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[x], fb[y], acc[x][y], 0, 0, 0);
      }
    }
    if (s + 1 < nst) {
      la.store(lds[buf ^ 1][0], ar, ah);
      lb.store(lds[buf ^ 1][1], br, bh);
    }
    __syncthreads();
  }

  // epilogue: lane l, register r of block (x, y) holds output
  //   i = i0 + wm*64 + x*32 + 8*(r/4) + 4*(l/32) + r%4,  j = j0 + wn*64 + y*32 + l%32.
  // Half a tile (the 64 columns of the waves with wn == half) is staged in LDS per pass.
  float *stage = (float *)smem;
  float mx = 0.f;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (wn == half) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int il = wm * 64 + x * 32 + 8 * g + 4 * (lane >> 5), jl = y * 32 + (lane & 31);
            *(float4 *)(stage + jl * kStageLd + il) =
                make_float4(acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
          }
    }
    __syncthreads();
    mx = fmaxf(mx, epilogue_block<kThreads>(e, stage, kStageLd, kBM, 64, i0, j0 + 64 * half, m, n));
    __syncthreads();
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int MODE, int AT, int BT>
hipError_t run(bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
               int k, const Epilogue &e, hipStream_t s) {
  const dim3 grid((n + kBN - 1) / kBN, (m + kBM - 1) / kBM);
#define E5MA_GG(AK, BK) gemm_generic_kernel<MODE, AT, BT, AK, BK><<<grid, kThreads, 0, s>>>(A, lda, B, ldb, m, n, k, e)
  if (akc && bkc) E5MA_GG(true, true);
  else if (akc) E5MA_GG(true, false);
  else if (bkc) E5MA_GG(false, true);
  else E5MA_GG(false, false);
#undef E5MA_GG
  return hipGetLastError();
}

template <int AT, int BT>
hipError_t pair(bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                int k, const Epilogue &e, hipStream_t s) {
  if constexpr (is_fp8(AT) && is_fp8(BT)) {
    if (mode_of(AT, BT, k) == kModeF8) return run<kModeF8, AT, BT>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    return run<kModeH, AT, BT>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  } else {
    return run<mode_of(AT, BT, 0), AT, BT>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  }
}

template <int AT>
hipError_t pair_b(int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m,
                  int n, int k, const Epilogue &e, hipStream_t s) {
  switch (bt) {
    case E5MA_E5M2: return pair<AT, E5MA_E5M2>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    case E5MA_E4M3: return pair<AT, E5MA_E4M3>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    case E5MA_BF16: return pair<AT, E5MA_BF16>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    default: return pair<AT, E5MA_FP32>(akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  }
}

}  // namespace

hipError_t launch_gemm_generic(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                               long long ldb, int m, int n, int k, const Epilogue &e, hipStream_t s) {
  switch (at) {
    case E5MA_E5M2: return pair_b<E5MA_E5M2>(bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    case E5MA_E4M3: return pair_b<E5MA_E4M3>(bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    case E5MA_BF16: return pair_b<E5MA_BF16>(bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
    default: return pair_b<E5MA_FP32>(bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
  }
}

}  // namespace e5ma
