// gemm_f8_kernel.hpp -- the fast FP8 x FP8 path of e5ma_gemm, for every operand layout: each of A and
// B is either K-contiguous (transa = T / transb = N, the cuBLASLt / TE forward layout) or
// M / N-contiguous (transa = N / transb = T: TE's dgrad and wgrad), k a multiple of 256 and
// k >= kF8MinK (the accuracy threshold of the FP8 matrix cores, gemm_common.hpp).  Replaces the
// reference's FFMA tile loop (src/gemm_e5m2effma.cuh:117-233) for these cases.  Included by one
// translation unit per layout pair (gemm_f8_tn/nn/nt/tt.hip), which build in parallel.
//
// Block tile 256 x 256, 4 waves (one per SIMD), each owning a 128 x 128 sub-tile held as 4 x 4
// accumulator blocks of v_mfma_f32_32x32x64_f8f6f4 (256 accumulator registers per lane).
// K advances in stages of 64 bytes.  A 4-slot LDS ring (4 x 32 KiB, one object per slot and operand)
// is filled by direct-to-LDS loads (global_load_lds_dwordx4: 64 lanes x 16 bytes land contiguously,
// no VGPR staging) issued three stages ahead; each stage costs one barrier.  The loads address a stage
// as a scalar base (advanced per stage) plus per-lane offsets fixed for the whole K loop, so the loop
// issues no vector ALU instructions besides the MFMAs.  The fragments are
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
#include "gemm_tile.hpp"

namespace e5ma {
namespace {
namespace f8k {

using namespace tile;

constexpr int kBK = 64;                            // K bytes (= elements) per stage
constexpr int kSlots = 4;                          // LDS ring depth (3 stages in flight)
constexpr int kOpBytes = kBM * kBK;                // 16 KiB per operand and stage
constexpr int kLoadsPerWave = kOpBytes / 1024 / 4; // dwordx4 LDS loads per wave, operand and stage

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// Per-lane byte offset, from the operand's stage base, of this lane's 16 bytes in the 1 KiB
// direct-to-LDS load blk (of 16) of an operand stage.  Stage s's base is P + r0 * ld + s * kBK for a
// K-contiguous operand and P + r0 + s * kBK * ld for an M / N-contiguous one, so the offsets are the
// same for every stage.
// K-contiguous: rows r0 + 16 blk .. + 15, 64 K bytes each (rows past lim repeat row lim - 1); 16-byte
// chunk c of row r lands at chunk c ^ swz(r).
// M / N-contiguous: k-rows 4 blk .. + 3 of the stage, 256 bytes of rows r0 .. r0 + 255 each (chunks
// past lim, a multiple of 16, repeat the last chunk; never stored).
// Offsets stay below 2^32 for ld <= kMaxLd (checked by the host).
template <bool KC> __device__ __forceinline__ uint32_t op_offset(long long ld, int lim, int r0, int blk, int lane) {
  if constexpr (KC) {
    const int r = blk * 16 + (lane >> 2);
    const int c = (lane & 3) ^ swz(r);
    return (uint32_t)(min(r0 + r, lim - 1) - r0) * (uint32_t)ld + 16 * c;
  } else {
    const int kk = blk * 4 + (lane >> 4);
    const int c = (lane & 15) ^ ((kk & 7) << 1);
    return (uint32_t)kk * (uint32_t)ld + (uint32_t)(min(r0 + 16 * c, lim - 16) - r0);
  }
}

// What the loads of one block need: the operands' stage-0 bases and per-stage strides (wave-uniform)
// and this lane's offsets for its share (kLoadsPerWave loads per operand and stage)
struct Loads {
  const uint8_t *a, *b;
  long long sa, sb;
  uint32_t oa[kLoadsPerWave], ob[kLoadsPerWave];
  uint32_t lds0;  // LDS offset of this wave's share within a buffer
};

template <bool AKC, bool BKC>
__device__ __forceinline__ Loads make_loads(const TileArgs &t, int i0, int j0, int wave, int lane) {
  Loads L;
  L.a = uniform_ptr(t.A + (AKC ? (long long)i0 * t.lda : i0));
  L.b = uniform_ptr(t.B + (BKC ? (long long)j0 * t.ldb : j0));
  L.sa = AKC ? kBK : kBK * t.lda;
  L.sb = BKC ? kBK : kBK * t.ldb;
#pragma unroll
  for (int q = 0; q < kLoadsPerWave; ++q) {
    L.oa[q] = op_offset<AKC>(t.lda, t.m, i0, wave * kLoadsPerWave + q, lane);
    L.ob[q] = op_offset<BKC>(t.ldb, t.n, j0, wave * kLoadsPerWave + q, lane);
  }
  L.lds0 = wave * kLoadsPerWave * 1024;
  return L;
}

// load q (of kLoadsPerWave) of this wave's share of stage s: 1 KiB of A and 1 KiB of B into LDS
// slot SLOT
template <int SLOT>
__device__ __forceinline__ void issue_load(const Loads &L, int s, int q) {
  load_lds16s(L.a + s * L.sa, L.oa[q], lds_addr(lds_a<SLOT>()) + L.lds0 + q * 1024);
  load_lds16s(L.b + s * L.sb, L.ob[q], lds_addr(lds_b<SLOT>()) + L.lds0 + q * 1024);
}
template <int SLOT>
__device__ __forceinline__ void issue_stage(const Loads &L, int s) {
#pragma unroll
  for (int q = 0; q < kLoadsPerWave; ++q) issue_load<SLOT>(L, s, q);
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

// Stage s (= SLOT mod 4) of the K loop.  The fragments are double-buffered by stage parity: set
// P = SLOT & 1 holds stage s's, and stage s + 1's are read into set 1 - P from the start of stage s, one
// fragment every second MFMA (LDS reads interleaved one per MFMA), so they have the whole stage to
// land.  (Single-buffered, the last reads of a stage were issued with its last MFMAs; slowed by the
// direct-to-LDS writes, they left the matrix cores idle at the barrier.)  WAITN: global loads this wave
// may leave in flight when stage s + 1 must have landed; NEXT: a stage s + 1 exists; ISSUE: stage s + 4
// exists.  The loads of stage s + 4 into stage s's slot (free: every wave read it before the barrier)
// go out one pair after every fourth MFMA.  (Issuing the 8 loads as one burst stalled the MFMA stream.)
template <int WAITN, bool NEXT, bool ISSUE, int SLOT, int AT, int BT, bool AKC, bool BKC>
__device__ __forceinline__ void f8_stage(const Loads &L, int s, int lane, int wm, int wn, v8i (&a)[2][4],
                                         v8i (&b)[2][4], v16f (&acc)[4][4]) {
  constexpr int P = SLOT & 1, Q = P ^ 1;
  if constexpr (NEXT) wait_barrier<WAITN>();
  const uint8_t *na = lds_a<(SLOT + 1) & 3>(), *nb = lds_b<(SLOT + 1) & 3>();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      // scale operands 0 select the unscaled v_mfma_f32_32x32x64_f8f6f4 (same products as the scaled form
      // with the neutral scale 127, one instruction dword pair shorter)
      acc[x][y] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[P][x], b[P][y], acc[x][y], kMfmaFmt<AT>,
                                                                  kMfmaFmt<BT>, 0, 0, 0, 0);
      if constexpr (ISSUE) {
        if (y == 1) issue_load<SLOT>(L, s + 4, x);
      }
      if constexpr (NEXT) {
        const int i = 4 * x + y;  // fragment i / 2 of the next stage after MFMA i (i even)
        if ((i & 1) == 0) {
          const int f = i >> 1;
          if (f < 4) a[Q][f] = read_frag<AKC>(na, 128 * wm + 32 * f, lane);
          else b[Q][f - 4] = read_frag<BKC>(nb, 128 * wn + 32 * (f - 4), lane);
        }
      }
    }
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

template <int AT, int BT, int DT, bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads, 1) void gemm_f8_kernel(TileArgs t, Epilogue e, int simple, int vec) {
  __shared__ float red[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn, sp;
  tile_of(blockIdx.x, t, tm, tn, sp);
  apply_split(t, e, sp);
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
  const Loads L = make_loads<AKC, BKC>(t, i0, j0, wave, lane);
  issue_stage<0>(L, 0);
  issue_stage<1>(L, 1);
  issue_stage<2>(L, 2);
  wait_barrier<2 * 2 * kLoadsPerWave>();  // stage 0 landed; stages 1 and 2 may be in flight
  issue_stage<3>(L, 3);
  v8i a[2][4], b[2][4];  // fragments, double-buffered by stage parity
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a[0][x] = read_frag<AKC>(lds_a<0>(), 128 * wm + 32 * x, lane);
    b[0][x] = read_frag<BKC>(lds_b<0>(), 128 * wn + 32 * x, lane);
  }
  // steady state, four stages (one per ring slot) per iteration: stages s + 2 and s + 3 in flight
  // while s + 1 is awaited; then the last four stages drain the ring (nk % 4 == 0)
  constexpr int kW2 = 2 * 2 * kLoadsPerWave, kW1 = 2 * kLoadsPerWave;
  int s = 0;
  for (; s < nk - 4; s += 4) {
    f8_stage<kW2, true, true, 0, AT, BT, AKC, BKC>(L, s, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 1, AT, BT, AKC, BKC>(L, s + 1, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 2, AT, BT, AKC, BKC>(L, s + 2, lane, wm, wn, a, b, acc);
    f8_stage<kW2, true, true, 3, AT, BT, AKC, BKC>(L, s + 3, lane, wm, wn, a, b, acc);
  }
  f8_stage<kW2, true, false, 0, AT, BT, AKC, BKC>(L, s, lane, wm, wn, a, b, acc);
  f8_stage<kW1, true, false, 1, AT, BT, AKC, BKC>(L, s + 1, lane, wm, wn, a, b, acc);
  f8_stage<0, true, false, 2, AT, BT, AKC, BKC>(L, s + 2, lane, wm, wn, a, b, acc);
  f8_stage<0, false, false, 3, AT, BT, AKC, BKC>(L, s + 3, lane, wm, wn, a, b, acc);

  const float mx = tile_epilogue<DT>(t, e, acc, i0, j0, wm, wn, lane, tid, simple, vec);
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

template <int AT, int BT, bool AKC, bool BKC>
hipError_t run_d(const TileArgs &t, const Epilogue &e, hipStream_t s) {
  const int grid = t.tiles_m * t.tiles_n * t.splits;
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

// every FP8 pairing for one layout pair; with splits > 1, k is split into equal parts and e describes
// the FP32 partial output of split 0 (the next split's follows at e.ldd * n floats)
template <bool AKC, bool BKC>
hipError_t launch_layout(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                         int k, int splits, const Epilogue &e, hipStream_t s) {
  const int ks = k / splits;
  TileArgs t{A, B, lda, ldb, m, n, ks, (m + kBM - 1) / kBM, (n + kBN - 1) / kBN, splits,
             AKC ? ks : ks * lda, BKC ? ks : ks * ldb, e.ldd * n * 4};
  if (at == E5MA_E5M2) return bt == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_E5M2, AKC, BKC>(t, e, s) : run_d<E5MA_E5M2, E5MA_E4M3, AKC, BKC>(t, e, s);
  return bt == E5MA_E5M2 ? run_d<E5MA_E4M3, E5MA_E5M2, AKC, BKC>(t, e, s) : run_d<E5MA_E4M3, E5MA_E4M3, AKC, BKC>(t, e, s);
}

}  // namespace f8k
}  // namespace
}  // namespace e5ma
