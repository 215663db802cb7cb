// gemm_f8.hip -- the fast FP8 x FP8 path of e5ma_gemm: both operands K-contiguous (transa = T,
// transb = N, the cuBLASLt / TE FP8 layout), k a multiple of 64 and k >= kF8MinK (the accuracy
// threshold of the FP8 matrix cores, gemm_common.hpp).  Replaces the reference's FFMA tile loop
// (src/gemm_e5m2effma.cuh:117-233) for this case.
//
// Block tile 256 x 256, 4 waves (one per SIMD), each owning a 128 x 128 sub-tile held as 4 x 4
// accumulator blocks of v_mfma_scale_f32_32x32x64_f8f6f4 (256 accumulator registers per lane).
// K advances in stages of 64 bytes.  A 4-slot LDS ring (4 x 32 KiB, one object per slot and operand)
// is filled by direct-to-LDS loads (global_load_lds_dwordx4: 64 lanes x 16 bytes land contiguously,
// no VGPR staging) issued three stages ahead; each stage costs one barrier.  The fragments are
// single-buffered (64 VGPRs beside the 256 accumulator registers) and the stage loop is unrolled by 4
// so that ring slots are compile-time indices.  Within a stage the MFMAs, the fragment reads of the
// next stage and the loads of stage s + 4 are interleaved.  LDS rows are 64 bytes; 16-byte chunk c of
// row r is stored at chunk c ^ ((r >> 2) & 3): gfx950's LDS serves a ds_read_b128 16 lanes per
// cycle over 64 banks (measured: a contiguous read takes 4 cycles, lanes l and l + 8 share a cycle,
// l and l + 16 do not), and with this swizzle the fragment reads are conflict-free (measured).
// Tiles are ordered so that the 32 blocks an XCD runs at once form a 4 x 8 patch of the output
// (A slices shared by 8 blocks, B slices by 4, in that XCD's L2).
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {
namespace {

using namespace dev;
using namespace gemm;

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256;
constexpr int kSlots = 4;                         // LDS ring depth (3 stages in flight)
constexpr int kOpBytes = kBM * kBK;               // 16 KiB per operand and stage
constexpr int kLoadsPerWave = kOpBytes / 1024 / 4; // dwordx4 LDS loads per wave, operand and stage
constexpr int kGroupM = 4;                        // tile order: groups of 4 m-tiles

typedef __attribute__((address_space(3))) void lds_void;

// The LDS ring as 8 distinct objects (slot x operand): with a separate object per slot the compiler's
// wait-count pass can tell that the fragment reads of one slot do not alias the direct-to-LDS loads
// still in flight into the others, and does not wait for those loads.
__shared__ __attribute__((aligned(1024))) uint8_t g_sa0[kOpBytes], g_sa1[kOpBytes], g_sa2[kOpBytes], g_sa3[kOpBytes];
__shared__ __attribute__((aligned(1024))) uint8_t g_sb0[kOpBytes], g_sb1[kOpBytes], g_sb2[kOpBytes], g_sb3[kOpBytes];
template <int S> __device__ __forceinline__ uint8_t *lds_a() {
  if constexpr (S == 0) return g_sa0; else if constexpr (S == 1) return g_sa1; else if constexpr (S == 2) return g_sa2;
  else return g_sa3;
}
template <int S> __device__ __forceinline__ uint8_t *lds_b() {
  if constexpr (S == 0) return g_sb0; else if constexpr (S == 1) return g_sb1; else if constexpr (S == 2) return g_sb2;
  else return g_sb3;
}
typedef __attribute__((address_space(1))) const void glob_cvoid;

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// s_waitcnt vmcnt(N) lgkmcnt(0), then s_barrier; the memory clobber keeps the compiler from moving
// memory operations across it.  (__syncthreads would also wait for every outstanding global load.)
template <int N> __device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

struct TileArgs {
  const uint8_t *A, *B;
  long long lda, ldb;
  int m, n, k;
  int tiles_m, tiles_n;
};

// output tile of block b: XCD-aware when the tile count is a multiple of 8 (blocks are dispatched to
// the 8 XCDs round-robin), then grouped kGroupM m-tiles at a time
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  int t = b;
  if ((total & 7) == 0) t = (b & 7) * (total >> 3) + (b >> 3);
  const int per_group = kGroupM * tiles_n;
  const int g = t / per_group, r = t - g * per_group;
  const int gm = min(kGroupM, tiles_m - g * kGroupM);
  tm = g * kGroupM + r % gm;
  tn = r / gm;
}

// One direct-to-LDS load: 16 bytes per lane from src land at lds + 16 * lane (lds wave-uniform).
// Written as inline asm so that the compiler's wait-count pass does not treat it as an LDS store it
// must wait for before every later LDS read: this kernel orders the ring slots itself (wait_barrier
// with explicit vmcnt).  Vector-memory operations complete in issue order, so these extra loads in
// flight can only make a wait the compiler emits for its own loads more conservative.  It sets m0
// itself; the compiler emits no other m0 use in this file (checked in the generated code).
__device__ __forceinline__ void load_lds16(const uint8_t *src, const uint8_t *lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "memory", "m0");
}

// load q (of kLoadsPerWave) of this wave's share of one stage: 1 KiB of A rows and 1 KiB of B rows
// (16 rows each) into LDS slot SLOT
template <int SLOT>
__device__ __forceinline__ void issue_load(const TileArgs &t, int kb, int i0, int j0, int wave, int lane, int q) {
  const int blk = wave * kLoadsPerWave + q;
  const int r = blk * 16 + (lane >> 2);
  const int c = (lane & 3) ^ swz(r);
  const int ra = min(i0 + r, t.m - 1), rb = min(j0 + r, t.n - 1);
  load_lds16(t.A + (long long)ra * t.lda + kb + 16 * c, lds_a<SLOT>() + blk * 1024);
  load_lds16(t.B + (long long)rb * t.ldb + kb + 16 * c, lds_b<SLOT>() + blk * 1024);
}
template <int SLOT> __device__ __forceinline__ void issue_stage(const TileArgs &t, int kb, int i0, int j0, int wave,
                                                               int lane) {
#pragma unroll
  for (int q = 0; q < kLoadsPerWave; ++q) issue_load<SLOT>(t, kb, i0, j0, wave, lane, q);
}

// fragments of one 32-row block of an operand stage: lane l holds the 32 K bytes
// [32 * (l / 32), + 32) of row r0 + l % 32
__device__ __forceinline__ v8i read_frag(const uint8_t *s, int r0, int lane) {
  const int r = r0 + (lane & 31);
  const int c0 = 2 * (lane >> 5);
  const uint8_t *row = s + r * kBK;
  const uint4 lo = *(const uint4 *)(row + 16 * (c0 ^ swz(r)));
  const uint4 hi = *(const uint4 *)(row + 16 * ((c0 + 1) ^ swz(r)));
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// Stage s (= SLOT mod 4) of the K loop; a / b hold stage s's fragments.  WAITN: global loads this
// wave may leave in flight when stage s + 1 must have landed; NEXT: a stage s + 1 exists; ISSUE:
// stage s + 4 exists.  After the barrier the 16 MFMAs of stage s are issued; the loads of stage s + 4
// into stage s's slot (free: every wave read it before the barrier) go out one pair after every
// fourth MFMA, and each fragment register is refilled from stage s + 1 right after its last use, with
// the LDS reads spread one per MFMA.  (Issuing the 8 loads as one burst stalled the MFMA stream.)
template <int WAITN, bool NEXT, bool ISSUE, int SLOT, int AT, int BT>
__device__ __forceinline__ void f8_stage(const TileArgs &t, int s, int i0, int j0, int wave, int lane, int wm, int wn,
                                         v8i (&a)[4], v8i (&b)[4], v16f (&acc)[4][4]) {
  if constexpr (NEXT) wait_barrier<WAITN>();
  const uint8_t *na = lds_a<(SLOT + 1) & 3>(), *nb = lds_b<(SLOT + 1) & 3>();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      acc[x][y] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[x], b[y], acc[x][y], kMfmaFmt<AT>, kMfmaFmt<BT>, 0,
                                                                  kNeutralScale, 0, kNeutralScale);
      if constexpr (ISSUE) {
        if (y == 1) issue_load<SLOT>(t, (s + 4) * kBK, i0, j0, wave, lane, x);
      }
      if constexpr (NEXT) {
        if (x == 3) b[y] = read_frag(nb, 128 * wn + 32 * y, lane);
      }
    }
    if constexpr (NEXT) a[x] = read_frag(na, 128 * wm + 32 * x, lane);
  }
  if constexpr (NEXT) {
    // keep the LDS reads spread over the MFMA stream: MFMA, DS read, MFMA, DS read, ...
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
}

template <int AT, int BT, int DT>
__global__ __launch_bounds__(kThreads, 1) void gemm_f8_tn_kernel(TileArgs t, Epilogue e, int simple, int vec_store) {
  __shared__ float red[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_of(blockIdx.x, t.tiles_m, t.tiles_n, tm, tn);
  const int i0 = tm * kBM, j0 = tn * kBN;
  const int nk = t.k / kBK;

  v16f acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  // prologue: stages 0..2 in flight; stage 3 is issued once every wave is past the first barrier
  issue_stage<0>(t, 0 * kBK, i0, j0, wave, lane);
  issue_stage<1>(t, 1 * kBK, i0, j0, wave, lane);
  issue_stage<2>(t, 2 * kBK, i0, j0, wave, lane);
  wait_barrier<2 * 2 * kLoadsPerWave>();  // stage 0 landed; stages 1 and 2 may be in flight
  issue_stage<3>(t, 3 * kBK, i0, j0, wave, lane);
  v8i a[4], b[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a[x] = read_frag(lds_a<0>(), 128 * wm + 32 * x, lane);
    b[x] = read_frag(lds_b<0>(), 128 * wn + 32 * x, lane);
  }
  // steady state, four stages (one per ring slot) per iteration: stages s + 2 and s + 3 in flight
  // while s + 1 is awaited; then the last four stages drain the ring (nk % 4 == 0)
  constexpr int kW2 = 2 * 2 * kLoadsPerWave, kW1 = 2 * kLoadsPerWave;
  int s = 0;
  for (; s < nk - 4; s += 4) {
    f8_stage<kW2, true, true, 0, AT, BT>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 1, AT, BT>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 2, AT, BT>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 3, AT, BT>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);
  }
  f8_stage<kW2, true, false, 0, AT, BT>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<kW1, true, false, 1, AT, BT>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<0, true, false, 2, AT, BT>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<0, false, false, 3, AT, BT>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);

  // ---- epilogue.  Lane l, register r of block (x, y): output
  //   i = i0 + 128*wm + 32*x + 8*(r/4) + 4*(l/32) + r%4,  j = j0 + 128*wn + 32*y + l%32
  float mx = 0.f;
  if (simple) {
    // no bias, beta = 0: scale, convert and store straight from the accumulators
    const EpiState st = epi_begin(e);
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int j = j0 + 128 * wn + 32 * y + (lane & 31);
      const float sbj = e.sb_vec ? e.sb[min(j, t.n - 1)] : 1.f;
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ib = i0 + 128 * wm + 32 * x + 8 * g + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float s = st.s;
            if (e.sa_vec || e.sb_vec) {
              const float sai = e.sa_vec ? e.sa[min(ib + q, t.m - 1)] : scale_or_one(e.sa);
              s = (e.alpha * sai) * (e.sb_vec ? sbj : scale_or_one(e.sb));
            }
            v[q] = acc[x][y][4 * g + q] * s;
          }
          if (j < t.n) {
            uint8_t *dp = (uint8_t *)e.d + ((size_t)j * e.ldd + ib) * elem_bytes(DT);
            if (vec_store && ib + 3 < t.m) {
              if constexpr (DT == E5MA_FP32) {
                *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
              } else if constexpr (is_fp8(DT)) {
                *(uint32_t *)dp = encode_t<DT>(v[0], st.qscale) | encode_t<DT>(v[1], st.qscale) << 8 |
                                  encode_t<DT>(v[2], st.qscale) << 16 | encode_t<DT>(v[3], st.qscale) << 24;
              } else {
                *(uint2 *)dp = make_uint2(encode_t<DT>(v[0], 1.f) | encode_t<DT>(v[1], 1.f) << 16,
                                          encode_t<DT>(v[2], 1.f) | encode_t<DT>(v[3], 1.f) << 16);
              }
#pragma unroll
              for (int q = 0; q < 4; ++q) mx = amax_fold(mx, v[q]);
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                if (ib + q < t.m) {
                  store_t<DT>(e.d, (size_t)j * e.ldd + ib + q, v[q], st.qscale);
                  mx = amax_fold(mx, v[q]);
                }
            }
          }
        }
    }
  } else {
    // bias and / or beta * C: stage 16 columns of accumulators at a time through LDS (slot 0 of the
    // ring, free now) and run the general epilogue along contiguous rows
    float *stage = (float *)lds_a<0>();
    constexpr int ld = kBM;
    __syncthreads();
    // pass p stages the 16 columns [16 p, + 16) of every 32-column accumulator block y of the waves
    // with wn == p / 2 ... all 256 rows: columns 128 * wn + 32 * y + 16 * (p & 1) + c, c < 16
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      const int pwn = pass >> 1, half = pass & 1;
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        __syncthreads();
        if (wn == pwn && ((lane & 31) >> 4) == half) {
#pragma unroll
          for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int il = 128 * wm + 32 * x + 8 * g + 4 * (lane >> 5), jl = lane & 15;
              *(float4 *)(stage + jl * ld + il) =
                  make_float4(acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
            }
        }
        __syncthreads();
        mx = fmaxf(mx, epilogue_block<kThreads>(e, stage, ld, kBM, 16, i0, j0 + 128 * pwn + 32 * y + 16 * half, t.m,
                                                t.n));
      }
    }
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int AT, int BT>
hipError_t run_d(const TileArgs &t, const Epilogue &e, hipStream_t s) {
  const int grid = t.tiles_m * t.tiles_n;
  const int simple = e.bias == nullptr && e.beta == 0.f;
  const int vec = ((uintptr_t)e.d % (4 * elem_bytes(e.d_dtype))) == 0 && e.ldd % 4 == 0;
#define E5MA_F8(DT) gemm_f8_tn_kernel<AT, BT, DT><<<grid, kThreads, 0, s>>>(t, e, simple, vec)
  switch (e.d_dtype) {
    case E5MA_BF16: E5MA_F8(E5MA_BF16); break;
    case E5MA_FP16: E5MA_F8(E5MA_FP16); break;
    case E5MA_FP32: E5MA_F8(E5MA_FP32); break;
    case E5MA_E5M2: E5MA_F8(E5MA_E5M2); break;
    default: E5MA_F8(E5MA_E4M3); break;
  }
#undef E5MA_F8
  return hipGetLastError();
}

}  // namespace

bool gemm_f8_tn_applies(int at, int bt, bool akc, bool bkc, int m, int n, int k) {
  // the K loop runs whole rounds of the 4-slot ring: k a multiple of 4 stages, at least 2 rounds
  return is_fp8(at) && is_fp8(bt) && akc && bkc && k % (kSlots * kBK) == 0 && k >= 2 * kSlots * kBK &&
         mode_of(at, bt, k) == kModeF8 && m > 0 && n > 0;
}

hipError_t launch_gemm_f8_tn(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m,
                             int n, int k, const Epilogue &e, hipStream_t s) {
  TileArgs t{A, B, lda, ldb, m, n, k, (m + kBM - 1) / kBM, (n + kBN - 1) / kBN};
  if (at == E5MA_E5M2) return bt == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_E5M2>(t, e, s) : run_d<E5MA_E5M2, E5MA_E4M3>(t, e, s);
  return bt == E5MA_E5M2 ? run_d<E5MA_E4M3, E5MA_E5M2>(t, e, s) : run_d<E5MA_E4M3, E5MA_E4M3>(t, e, s);
}

}  // namespace e5ma

