// gemm_f8_kernel.hpp -- the fast FP8 x FP8 path of e5ma_gemm, for every operand layout: each of A and
// B is either K-contiguous (transa = T / transb = N, the cuBLASLt / TE forward layout) or
// M / N-contiguous (transa = N / transb = T: TE's dgrad and wgrad), k a multiple of 256 and
// k >= kF8MinK (the accuracy threshold of the FP8 matrix cores, gemm_common.hpp).  Replaces the
// reference's FFMA tile loop (src/gemm_e5m2effma.cuh:117-233) for these cases.  Included by one
// translation unit per layout pair (gemm_f8_tn/nn/nt/tt.hip), which build in parallel.
//
// Block tile 256 x 256, 4 waves (one per SIMD), each owning a 128 x 128 sub-tile held as 4 x 4
// accumulator blocks of v_mfma_scale_f32_32x32x64_f8f6f4 (256 accumulator registers per lane).
// K advances in stages of 64 bytes.  A 4-slot LDS ring (4 x 32 KiB, one object per slot and operand)
// is filled by direct-to-LDS loads (global_load_lds_dwordx4: 64 lanes x 16 bytes land contiguously,
// no VGPR staging) issued three stages ahead; each stage costs one barrier.  The fragments are
// single-buffered (64 VGPRs beside the 256 accumulator registers) and the stage loop is unrolled by 4
// so that ring slots are compile-time indices.  Within a stage the MFMAs, the fragment reads of the
// next stage and the loads of stage s + 4 are interleaved.
//
// LDS layout of one operand stage (16 KiB), by source layout:
// - K-contiguous: 256 rows (m or n) of 64 K bytes; 16-byte chunk c of row r is stored at chunk
//   c ^ ((r >> 2) & 3).  gfx950's LDS serves a ds_read_b128 16 lanes per cycle over 64 banks
//   (measured: a contiguous read takes 4 cycles, lanes l and l + 8 share a cycle, l and l + 16 do
//   not); with this swizzle the fragment reads (2 x ds_read_b128 per lane) are conflict-free (measured).
// - M / N-contiguous: 64 K rows of 256 m (or n) bytes, as the global rows are; chunk c of k-row kk is
//   stored at chunk c ^ ((kk & 7) << 1).  Fragments are read with the transposing ds_read_b64_tr_b8
//   (4 per lane): within each group of 16 lanes, output lane 8h + t receives as its byte b the byte t
//   of the 8 bytes addressed by lane 2b + h (measured on gfx950).  Lanes 2b + h address k-row b of an
//   8-row group at rows (m) 8h..8h+7, so lane 8h + t gets 8 consecutive k of row 8h + t: the MFMA
//   fragment layout.  The swizzle puts the 8 k-rows x 2 halves of one group and the two groups of a
//   32-lane half on 16 distinct chunks, i.e. all 64 banks once.
// Tiles are ordered so that the 32 blocks an XCD runs at once form a 4 x 8 patch of the output
// (A slices shared by 8 blocks, B slices by 4, in that XCD's L2).
#pragma once
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
typedef __attribute__((address_space(3))) v2i lds_v2i;

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
// the ring's 8 buffers as the epilogue's 8 column groups of 16 FP32 columns x 256 rows (g is
// wave-uniform, or a constant after unrolling)
__device__ __forceinline__ float *stage_at(int g) {
  switch (g) {
    case 0: return (float *)lds_a<0>(); case 1: return (float *)lds_a<1>();
    case 2: return (float *)lds_a<2>(); case 3: return (float *)lds_a<3>();
    case 4: return (float *)lds_b<0>(); case 5: return (float *)lds_b<1>();
    case 6: return (float *)lds_b<2>(); default: return (float *)lds_b<3>();
  }
}

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// One accumulator element copied to a VGPR where it is used.  The "a" constraint keeps the value in
// its accumulator register; left to itself the compiler copies whole accumulator blocks to VGPRs at
// the end of the K loop and spills them.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

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

// one 1 KiB direct-to-LDS load of an operand stage: block blk (of 16) of the slot.
// K-contiguous source: rows r0 + 16 blk .. + 15, 64 K bytes each (rows past lim repeat row lim - 1).
// M / N-contiguous source: k-rows 4 blk .. + 3 of the stage, 256 bytes of rows r0 .. r0 + 255 each
// (chunks past lim, a multiple of 16, repeat the last chunk; never stored).
template <bool KC>
__device__ __forceinline__ void load_op(const uint8_t *P, long long ld, int lim, int kb, int r0, int blk, int lane,
                                        uint8_t *lds) {
  if constexpr (KC) {
    const int r = blk * 16 + (lane >> 2);
    const int c = (lane & 3) ^ swz(r);
    load_lds16(P + (long long)min(r0 + r, lim - 1) * ld + kb + 16 * c, lds + blk * 1024);
  } else {
    const int kk = blk * 4 + (lane >> 4);
    const int c = (lane & 15) ^ ((kk & 7) << 1);
    load_lds16(P + (long long)(kb + kk) * ld + min(r0 + 16 * c, lim - 16), lds + blk * 1024);
  }
}

// load q (of kLoadsPerWave) of this wave's share of one stage: 1 KiB of A and 1 KiB of B into LDS
// slot SLOT
template <int SLOT, bool AKC, bool BKC>
__device__ __forceinline__ void issue_load(const TileArgs &t, int kb, int i0, int j0, int wave, int lane, int q) {
  const int blk = wave * kLoadsPerWave + q;
  load_op<AKC>(t.A, t.lda, t.m, kb, i0, blk, lane, lds_a<SLOT>());
  load_op<BKC>(t.B, t.ldb, t.n, kb, j0, blk, lane, lds_b<SLOT>());
}
template <int SLOT, bool AKC, bool BKC>
__device__ __forceinline__ void issue_stage(const TileArgs &t, int kb, int i0, int j0, int wave, int lane) {
#pragma unroll
  for (int q = 0; q < kLoadsPerWave; ++q) issue_load<SLOT, AKC, BKC>(t, kb, i0, j0, wave, lane, q);
}

// fragments of one 32-row block of an operand stage: lane l holds the 32 K bytes
// [32 * (l / 32), + 32) of row r0 + l % 32 (r0 a multiple of 32)
template <bool KC> __device__ __forceinline__ v8i read_frag(const uint8_t *s, int r0, int lane) {
  if constexpr (KC) {
    const int r = r0 + (lane & 31);
    const int c0 = 2 * (lane >> 5);
    const uint8_t *row = s + r * kBK;
    const uint4 lo = *(const uint4 *)(row + 16 * (c0 ^ swz(r)));
    const uint4 hi = *(const uint4 *)(row + 16 * ((c0 + 1) ^ swz(r)));
    return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  } else {
    // this lane addresses k-row 32 (g / 2) + 8 q + b, rows r .. r + 7 (r = r0 + 16 (g % 2) + 8 h) for
    // read q; it receives row r0 + l % 32, k 32 (l / 32) + 8 q .. + 7
    const int g = lane >> 4, h = lane & 1, b = (lane & 15) >> 1;
    const int r = r0 + 16 * (g & 1) + 8 * h;
    const uint8_t *p = s + (32 * (g >> 1) + b) * kBM + 16 * ((r >> 4) ^ (b << 1)) + (r & 15);
    const v2i q0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 0 * 8 * kBM));
    const v2i q1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 1 * 8 * kBM));
    const v2i q2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 2 * 8 * kBM));
    const v2i q3 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 3 * 8 * kBM));
    return v8i{q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
  }
}

// Stage s (= SLOT mod 4) of the K loop; a / b hold stage s's fragments.  WAITN: global loads this
// wave may leave in flight when stage s + 1 must have landed; NEXT: a stage s + 1 exists; ISSUE:
// stage s + 4 exists.  After the barrier the 16 MFMAs of stage s are issued; the loads of stage s + 4
// into stage s's slot (free: every wave read it before the barrier) go out one pair after every
// fourth MFMA, and each fragment register is refilled from stage s + 1 right after its last use, with
// the LDS reads spread one per MFMA.  (Issuing the 8 loads as one burst stalled the MFMA stream.)
template <int WAITN, bool NEXT, bool ISSUE, int SLOT, int AT, int BT, bool AKC, bool BKC>
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
        if (y == 1) issue_load<SLOT, AKC, BKC>(t, (s + 4) * kBK, i0, j0, wave, lane, x);
      }
      if constexpr (NEXT) {
        if (x == 3) b[y] = read_frag<BKC>(nb, 128 * wn + 32 * y, lane);
      }
    }
    if constexpr (NEXT) a[x] = read_frag<AKC>(na, 128 * wm + 32 * x, lane);
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

// Writes out one staged half tile (256 rows x 128 columns starting at column jh) in the reference's
// epilogue order (include/e5m2effma.h: v = acc * (alpha * sa[i]) * sb[j]; v += bias[i];
// v = fma(beta, C * csinv, v); amax; convert).  Wave w takes columns w, w + 4, ..., thread t rows
// i .. i + 3 (i = i0 + 4 (t % 64)); four columns per step, with their C values loaded before any is
// computed or stored, so 16 loads per thread are in flight (C may alias D: each element is read before
// it is written, by the same thread).  CT: the dtype of C, or -1 when beta = 0.
template <int DT, int CT>
__device__ __forceinline__ float general_half(const Epilogue &e, const EpiState &st, const TileArgs &t, int i, int jh,
                                              const float (&rs)[4], const float (&rb)[4], int vec, int tid,
                                              float mx) {
  const int w = tid >> 6, il = 4 * (tid & 63);
  const bool rows4 = i + 3 < t.m;
  const float sb1 = scale_or_one(e.sb);
#pragma unroll 1
  for (int c0 = 0; c0 < 32; c0 += 4) {
    float a[4][4], cv[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int jl = w + 4 * (c0 + u), j = jh + jl;
      const float4 v4 = *(const float4 *)(stage_at(jl >> 4) + (jl & 15) * kBM + il);
      a[u][0] = v4.x; a[u][1] = v4.y; a[u][2] = v4.z; a[u][3] = v4.w;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cv[u][q] = 0.f;
        if constexpr (CT >= 0) {
          if (j < t.n && i + q < t.m) cv[u][q] = load_t<CT>(e.c, (size_t)j * e.ldc + i + q, st.csinv);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = jh + w + 4 * (c0 + u);
      if (j >= t.n) continue;
      const float sbj = e.sb_vec ? e.sb[j] : sb1;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = a[u][q] * ((e.sa_vec || e.sb_vec) ? rs[q] * sbj : st.s);
        if (e.bias) v[q] = v[q] + rb[q];
        if constexpr (CT >= 0) v[q] = __builtin_fmaf(e.beta, cv[u][q], v[q]);
      }
      const size_t o = (size_t)j * e.ldd + i;
      if (rows4 && vec) {
        uint8_t *dp = (uint8_t *)e.d + o * elem_bytes(DT);
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
          if (i + q < t.m) {
            store_t<DT>(e.d, o + q, v[q], st.qscale);
            mx = amax_fold(mx, v[q]);
          }
      }
    }
  }
  return mx;
}

template <int AT, int BT, int DT, bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads, 1) void gemm_f8_kernel(TileArgs t, Epilogue e, int simple, int vec) {
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
  issue_stage<0, AKC, BKC>(t, 0 * kBK, i0, j0, wave, lane);
  issue_stage<1, AKC, BKC>(t, 1 * kBK, i0, j0, wave, lane);
  issue_stage<2, AKC, BKC>(t, 2 * kBK, i0, j0, wave, lane);
  wait_barrier<2 * 2 * kLoadsPerWave>();  // stage 0 landed; stages 1 and 2 may be in flight
  issue_stage<3, AKC, BKC>(t, 3 * kBK, i0, j0, wave, lane);
  v8i a[4], b[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a[x] = read_frag<AKC>(lds_a<0>(), 128 * wm + 32 * x, lane);
    b[x] = read_frag<BKC>(lds_b<0>(), 128 * wn + 32 * x, lane);
  }
  // steady state, four stages (one per ring slot) per iteration: stages s + 2 and s + 3 in flight
  // while s + 1 is awaited; then the last four stages drain the ring (nk % 4 == 0)
  constexpr int kW2 = 2 * 2 * kLoadsPerWave, kW1 = 2 * kLoadsPerWave;
  int s = 0;
  for (; s < nk - 4; s += 4) {
    f8_stage<kW2, true, true, 0, AT, BT, AKC, BKC>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 1, AT, BT, AKC, BKC>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 2, AT, BT, AKC, BKC>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 3, AT, BT, AKC, BKC>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);
  }
  f8_stage<kW2, true, false, 0, AT, BT, AKC, BKC>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<kW1, true, false, 1, AT, BT, AKC, BKC>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<0, true, false, 2, AT, BT, AKC, BKC>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
  f8_stage<0, false, false, 3, AT, BT, AKC, BKC>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);

  // ---- epilogue.  Lane l, register r of block (x, y): output
  //   i = i0 + 128*wm + 32*x + 8*(r/4) + 4*(l/32) + r%4,  j = j0 + 128*wn + 32*y + l%32
  // (scheduling barriers keep the compiler from hoisting epilogue work into the K loop's tail and from
  // copying all accumulators to VGPRs at once, both of which spill)
  __builtin_amdgcn_sched_barrier(0);
  float mx = 0.f;
  if (simple && i0 + kBM <= t.m && j0 + kBN <= t.n) {
    // no bias, beta = 0, a full tile, D aligned for 4-element stores: scale, convert and store straight
    // from the accumulators (no tail branches, so every loop unrolls and the accumulators stay in
    // registers)
    const EpiState st = epi_begin(e);
    const int ib0 = i0 + 128 * wm + 4 * (lane >> 5);
    const float sa1 = e.alpha * scale_or_one(e.sa), sb1 = scale_or_one(e.sb);
    // column by column (y outer): the 16 stores into one column's cache lines follow each other, so
    // the L2 writes the lines back whole (x / g outer measured 3x the write traffic)
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int j = j0 + 128 * wn + 32 * y + (lane & 31);
      const float sbj = e.sb_vec ? e.sb[j] : sb1;
      uint8_t *colp = (uint8_t *)e.d + ((size_t)j * e.ldd + ib0) * elem_bytes(DT);
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          __builtin_amdgcn_sched_barrier(0);
          const int ib = ib0 + 32 * x + 8 * g;
          float as[4];  // alpha * sa[i] of these 4 rows (OUTER scaling of A)
          if (e.sa_vec) {
            const float4 v = *(const float4 *)(e.sa + ib);
            as[0] = e.alpha * v.x; as[1] = e.alpha * v.y; as[2] = e.alpha * v.z; as[3] = e.alpha * v.w;
          } else {
            as[0] = as[1] = as[2] = as[3] = sa1;
          }
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float sc = (e.sa_vec || e.sb_vec) ? as[q] * sbj : st.s;
            v[q] = acc_read(acc[x][y][4 * g + q]) * sc;
            mx = amax_fold(mx, v[q]);
          }
          uint8_t *dp = colp + (32 * x + 8 * g) * elem_bytes(DT);
          if constexpr (DT == E5MA_FP32) {
            *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
          } else if constexpr (is_fp8(DT)) {
            *(uint32_t *)dp = encode_t<DT>(v[0], st.qscale) | encode_t<DT>(v[1], st.qscale) << 8 |
                              encode_t<DT>(v[2], st.qscale) << 16 | encode_t<DT>(v[3], st.qscale) << 24;
          } else {
            *(uint2 *)dp = make_uint2(encode_t<DT>(v[0], 1.f) | encode_t<DT>(v[1], 1.f) << 16,
                                      encode_t<DT>(v[2], 1.f) | encode_t<DT>(v[3], 1.f) << 16);
          }
        }
    }
  } else {
    // general epilogue (bias, beta * C, tails): half a tile at a time -- the 128 columns of the waves
    // with wn == h, 256 x 128 FP32 = the whole ring, column group c (16 columns) in ring buffer c --
    // is staged in LDS, then the block writes it out (general_half)
    const EpiState st = epi_begin(e);
    const int i = i0 + 4 * (tid & 63);  // this thread's 4 rows in the write-out
    float rs[4], rb[4];                 // alpha * sa[i], bias[i] of those rows
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int iq = min(i + q, t.m - 1);
      rs[q] = e.alpha * (e.sa_vec ? e.sa[iq] : scale_or_one(e.sa));
      rb[q] = e.bias ? load_any(e.bias_dtype, e.bias, (size_t)iq, 1.f) : 0.f;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __syncthreads();  // the ring (K loop) or the previous half is no longer read
      if (wn == h) {
#pragma unroll
        for (int y = 0; y < 4; ++y) {
          float *grp = (lane & 16) ? stage_at(2 * y + 1) : stage_at(2 * y);
          float *col = grp + (lane & 15) * kBM;
#pragma unroll
          for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int il = 128 * wm + 32 * x + 8 * g + 4 * (lane >> 5);
              *(float4 *)(col + il) = make_float4(acc_read(acc[x][y][4 * g]), acc_read(acc[x][y][4 * g + 1]),
                                                  acc_read(acc[x][y][4 * g + 2]), acc_read(acc[x][y][4 * g + 3]));
            }
        }
      }
      __syncthreads();
      const int c = e.beta != 0.f ? e.c_dtype : -1;
      if (c == E5MA_FP32) mx = general_half<DT, E5MA_FP32>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
      else if (c == E5MA_BF16) mx = general_half<DT, E5MA_BF16>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
      else if (c == E5MA_FP16) mx = general_half<DT, E5MA_FP16>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
      else if (c == E5MA_E5M2) mx = general_half<DT, E5MA_E5M2>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
      else if (c == E5MA_E4M3) mx = general_half<DT, E5MA_E4M3>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
      else mx = general_half<DT, -1>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
    }
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int AT, int BT, bool AKC, bool BKC>
hipError_t run_d(const TileArgs &t, const Epilogue &e, hipStream_t s) {
  const int grid = t.tiles_m * t.tiles_n;
  // the direct epilogue needs 4-element-aligned D columns and, with OUTER scaling of A, a 16-byte
  // aligned scale vector
  const int vec = ((uintptr_t)e.d % (4 * elem_bytes(e.d_dtype))) == 0 && e.ldd % 4 == 0 &&
                  (!e.sa_vec || (uintptr_t)e.sa % 16 == 0);
  const int simple = e.bias == nullptr && e.beta == 0.f && vec;
#define E5MA_F8(DT) gemm_f8_kernel<AT, BT, DT, AKC, BKC><<<grid, kThreads, 0, s>>>(t, e, simple, vec)
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

// every FP8 pairing for one layout pair
template <bool AKC, bool BKC>
hipError_t launch_layout(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                         int k, const Epilogue &e, hipStream_t s) {
  TileArgs t{A, B, lda, ldb, m, n, k, (m + kBM - 1) / kBM, (n + kBN - 1) / kBN};
  if (at == E5MA_E5M2)
    return bt == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_E5M2, AKC, BKC>(t, e, s) : run_d<E5MA_E5M2, E5MA_E4M3, AKC, BKC>(t, e, s);
  return bt == E5MA_E5M2 ? run_d<E5MA_E4M3, E5MA_E5M2, AKC, BKC>(t, e, s) : run_d<E5MA_E4M3, E5MA_E4M3, AKC, BKC>(t, e, s);
}

}  // namespace
}  // namespace e5ma
