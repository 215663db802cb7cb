// gemm_f8_kernel.hpp -- the fast FP8 x FP8 path of e5ma_gemm, for every operand layout: each of A and
// B is either K-contiguous (transa = T / transb = N, the cuBLASLt / TE forward layout) or
// M / N-contiguous (transa = N / transb = T: TE's dgrad and wgrad), k a multiple of 256 and
// k >= kF8MinK (the accuracy threshold of the FP8 matrix cores, gemm_common.hpp).  Replaces the
// reference's FFMA tile loop (src/gemm_e5m2effma.cuh:117-233) for these cases.  Included by one
// translation unit per layout pair (gemm_f8_tn/nn/nt/tt.hip), which build in parallel.
//
// Block tile 256 x 256, 4 waves (one per SIMD), each owning a 128 x 128 sub-tile held as 4 x 4
// accumulator blocks of v_mfma_f32_32x32x64_f8f6f4 (256 accumulator registers per lane).  K advances in
// units of 64 bytes (one MFMA K step: 16 MFMAs per wave); during each unit the next unit's fragments
// are read from LDS (double-buffered by unit parity, in the order its MFMAs use them).  The 128 KiB
// LDS ring is filled by direct-to-LDS loads (global_load_lds_dwordx4: 64 lanes x 16 bytes land
// contiguously, no VGPR staging) that address a stage as a scalar base (advanced per stage) plus
// per-lane offsets fixed for the whole K loop, so the loop issues no vector ALU instructions besides
// the MFMAs.  Two ring shapes (Ring<PAIR>), chosen by B's layout from measurements at 8192^3:
// - PAIR (B K-contiguous): 2 stages of 128 K bytes (2 x 64 KiB), two units each.  A K-contiguous
//   operand's rows are loaded 128 bytes (a whole cache line) per row and instruction: with 64-byte
//   stages every line was requested twice, half each time, which cost 11% of the TN GEMM's time.  One
//   barrier per stage, at its second unit: s_waitcnt vmcnt(0) lgkmcnt(0) completes this wave's loads
//   of stage p + 1 and its reads of stage p's region (the second unit's fragments, read during the
//   first), s_barrier makes both hold for every wave; then, during the second unit, stage p + 2's
//   loads go into that region, one pair (A, B) after every second MFMA.
// - 4 slots (B N-contiguous, whose rows are 256-byte k-rows either way): 4 stages of 64 K bytes, one
//   unit each, one barrier per unit.  Stage s + 3's loads go into slot (s + 3) % 4 = (s - 1) % 4, whose
//   last reads (stage s - 1's fragments) were issued during stage s - 2; the barrier starting stage s
//   waits with lgkmcnt(15), which completes those but not the ones of stage s - 1, issued just before.
//   One load pair goes out after every fourth MFMA.
// Either way a stage's loads have two units of MFMAs to land.
//
// LDS layout of one operand stage, by source layout:
// - K-contiguous: 256 rows (m or n) of kStageK K bytes; 16-byte chunk c of row r is stored at chunk
//   c ^ swz(r) (swz(r) = (r >> 1) & 7 for 128-byte rows, (r >> 2) & 3 for 64-byte rows).  gfx950's LDS
//   serves a ds_read_b128 16 lanes per cycle over 64 banks (measured: a contiguous read takes 4
//   cycles, lanes l and l + 8 share a cycle, l and l + 16 do not).  A fragment read has 16 consecutive
//   rows per cycle at one K chunk c; with 128-byte rows, rows 2u + v land on bank chunk 8v + (c ^ u),
//   with 64-byte rows rows 4v + w on 4w + (c ^ v): all 16 distinct, so the reads are conflict-free.
// - M / N-contiguous: kStageK K rows of 256 m (or n) bytes, as the global rows are; chunk c of k-row kk
//   is stored at chunk c ^ ((kk & 7) << 1).  Fragments are read with the transposing ds_read_b64_tr_b8
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

constexpr int kUnitK = 64;  // K bytes (= elements) of one MFMA step

template <bool PAIR> struct Ring {
  static constexpr int kStageK = PAIR ? 128 : 64;          // K bytes per stage
  static constexpr int kSlots = PAIR ? 2 : 4;              // stages the ring holds
  static constexpr int kOpBytes = kBM * kStageK;           // per operand and stage
  static constexpr int kLoads = kOpBytes / 1024 / 4;       // dwordx4 LDS loads per wave, operand and stage
  static constexpr int kLanesPerRow = kStageK / 16;        // K-contiguous: lanes loading one row
  static constexpr int kRowsPerLoad = 64 / kLanesPerRow;   // K-contiguous: rows per 1 KiB load
  static constexpr int kW1 = 2 * kLoads;                   // one stage's loads of A and B, per wave
  static_assert(kOpBytes * kSlots == 4 * kBufBytes, "the stages fill the ring");
  __device__ static int swz(int r) { return PAIR ? (r >> 1) & 7 : (r >> 2) & 3; }
  template <int S> __device__ static uint8_t *slot_a() { return lds_a<PAIR ? 2 * S : S>(); }
  template <int S> __device__ static uint8_t *slot_b() { return lds_b<PAIR ? 2 * S : S>(); }
};

// Per-lane byte offset, from the operand's stage base, of this lane's 16 bytes in the 1 KiB
// direct-to-LDS load blk of an operand stage.  Stage p's base is P + r0 * ld + p * kStageK for a
// K-contiguous operand and P + r0 + p * kStageK * ld for an M / N-contiguous one, so the offsets are
// the same for every stage.
// K-contiguous: rows r0 + kRowsPerLoad blk .., kStageK K bytes each (rows past lim repeat row lim - 1);
// lane l fetches chunk (l % kLanesPerRow) ^ swz(r) of its row, which lands at chunk l % kLanesPerRow.
// M / N-contiguous: k-rows 4 blk .. + 3 of the stage, 256 bytes of rows r0 .. r0 + 255 each (chunks
// past lim, a multiple of 16, repeat the last chunk; never stored).
// Offsets stay below 2^32 for ld <= kMaxLd (checked by the host).
template <bool KC, bool PAIR>
__device__ __forceinline__ uint32_t op_offset(long long ld, int lim, int r0, int blk, int lane) {
  using G = Ring<PAIR>;
  if constexpr (KC) {
    const int r = blk * G::kRowsPerLoad + lane / G::kLanesPerRow;
    const int c = (lane % G::kLanesPerRow) ^ G::swz(r);
    return (uint32_t)(min(r0 + r, lim - 1) - r0) * (uint32_t)ld + 16 * c;
  } else {
    const int kk = blk * 4 + (lane >> 4);
    const int c = (lane & 15) ^ ((kk & 7) << 1);
    return (uint32_t)kk * (uint32_t)ld + (uint32_t)(min(r0 + 16 * c, lim - 16) - r0);
  }
}

// What the loads of one block need: the operands' stage-0 bases and per-stage strides (wave-uniform)
// and this lane's offsets for its share (kLoads loads per operand and stage)
template <bool PAIR> struct Loads {
  const uint8_t *a, *b;
  long long sa, sb;
  uint32_t oa[Ring<PAIR>::kLoads], ob[Ring<PAIR>::kLoads];
  uint32_t lds0;  // LDS offset of this wave's share within a stage
};

template <bool AKC, bool BKC, bool PAIR>
__device__ __forceinline__ Loads<PAIR> make_loads(const TileArgs &t, int i0, int j0, int wave, int lane) {
  using G = Ring<PAIR>;
  Loads<PAIR> L;
  L.a = uniform_ptr(t.A + (AKC ? (long long)i0 * t.lda : i0));
  L.b = uniform_ptr(t.B + (BKC ? (long long)j0 * t.ldb : j0));
  L.sa = AKC ? G::kStageK : G::kStageK * t.lda;
  L.sb = BKC ? G::kStageK : G::kStageK * t.ldb;
#pragma unroll
  for (int q = 0; q < G::kLoads; ++q) {
    L.oa[q] = op_offset<AKC, PAIR>(t.lda, t.m, i0, wave * G::kLoads + q, lane);
    L.ob[q] = op_offset<BKC, PAIR>(t.ldb, t.n, j0, wave * G::kLoads + q, lane);
  }
  L.lds0 = wave * G::kLoads * 1024;
  return L;
}

// load q of this wave's share of stage p: 1 KiB of A and 1 KiB of B into ring slot S
template <int S, bool PAIR>
__device__ __forceinline__ void issue_load(const Loads<PAIR> &L, int p, int q) {
  using G = Ring<PAIR>;
  load_lds16s(L.a + p * L.sa, L.oa[q], lds_addr(G::template slot_a<S>()) + L.lds0 + q * 1024);
  load_lds16s(L.b + p * L.sb, L.ob[q], lds_addr(G::template slot_b<S>()) + L.lds0 + q * 1024);
}
template <int S, bool PAIR>
__device__ __forceinline__ void issue_stage(const Loads<PAIR> &L, int p) {
#pragma unroll
  for (int q = 0; q < Ring<PAIR>::kLoads; ++q) issue_load<S, PAIR>(L, p, q);
}

// fragments of one 32-row block of unit J of an operand stage: lane l holds the 32 K bytes
// [64 J + 32 * (l / 32), + 32) of row r0 + l % 32 (r0 a multiple of 32)
template <bool KC, bool PAIR, int J> __device__ __forceinline__ v8i read_frag(const uint8_t *s, int r0, int lane) {
  using G = Ring<PAIR>;
  if constexpr (KC) {
    const int r = r0 + (lane & 31);
    const int c0 = 4 * J + 2 * (lane >> 5);
    const uint8_t *row = s + r * G::kStageK;
    const uint4 lo = *(const uint4 *)(row + 16 * (c0 ^ G::swz(r)));
    const uint4 hi = *(const uint4 *)(row + 16 * ((c0 + 1) ^ G::swz(r)));
    return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  } else {
    // this lane addresses k-row 64 J + 32 (g / 2) + 8 q + b, rows r .. r + 7 (r = r0 + 16 (g % 2) + 8 h)
    // for read q; it receives row r0 + l % 32, k 64 J + 32 (l / 32) + 8 q .. + 7
    const int g = lane >> 4, h = lane & 1, b = (lane & 15) >> 1;
    const int r = r0 + 16 * (g & 1) + 8 * h;
    const uint8_t *p = s + (kUnitK * J + 32 * (g >> 1) + b) * kBM + 16 * ((r >> 4) ^ (b << 1)) + (r & 15);
    const v2i q0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 0 * 8 * kBM));
    const v2i q1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 1 * 8 * kBM));
    const v2i q2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 2 * 8 * kBM));
    const v2i q3 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + 3 * 8 * kBM));
    return v8i{q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
  }
}

// One unit: 4 NY MFMAs on fragment set P (NY = 4: a wave owns 128 x 128 of a 256 x 256 tile; NY = 2:
// 128 x 64 of a 256 x 128 half tile, accumulator blocks y < 2).
// BAR: wait_barrier<WAITN, LGK> after the first MFMA, before any LDS read or load of the unit.
// NEXT: the next unit's fragments (ring slot NS, unit NJ of that stage) are read into set 1 - P in the
//   order its MFMAs use them (its first NY need a0 and all of b): a0, b0 .. b(NY - 1), a1, a2, a3, one
//   every second MFMA (NY = 4) or every MFMA (NY = 2).
// ZERO: the tile's first unit, whose MFMAs take the inline constant 0 as their accumulator input (no
//   zeroing of 256 accumulator registers per tile).
// ISSUE: stage ls's loads go into ring slot IS, one pair (A, B) after every (4 NY / kLoads)-th MFMA.  A
//   half tile issues every load of a whole tile (the B rows it does not use included), so that every
//   wait count is the same for both widths.
template <bool PAIR, int P, bool BAR, int WAITN, int LGK, bool NEXT, int NS, int NJ, bool ISSUE, int IS, int AT,
          int BT, bool AKC, bool BKC, int NY, bool ZERO = false>
__device__ __forceinline__ void f8_unit(const Loads<PAIR> &L, int ls, int lane, int wm, int wn, v8i (&a)[2][4],
                                        v8i (&b)[2][4], v16f (&acc)[4][4]) {
  using G = Ring<PAIR>;
  constexpr int Q = 1 - P, kMf = 4 * NY, kEvery = kMf / G::kLoads, kAt = kEvery > 1 ? 1 : 0;
  constexpr int kFragStep = NY == 4 ? 2 : 1;  // MFMAs per fragment read
  static_assert(kMf % G::kLoads == 0, "whole loads per unit");
  const uint8_t *na = G::template slot_a<NS>(), *nb = G::template slot_b<NS>();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
#pragma unroll
    for (int y = 0; y < NY; ++y) {
      // scale operands 0 select the unscaled v_mfma_f32_32x32x64_f8f6f4 (same products as the scaled form
      // with the neutral scale 127, one instruction dword pair shorter)
      acc[x][y] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[P][x], b[P][y], ZERO ? v16f{} : acc[x][y],
                                                                  kMfmaFmt<AT>, kMfmaFmt<BT>, 0, 0, 0, 0);
      const int i = NY * x + y;
      if constexpr (BAR) {
        // the unit's barrier comes after its first MFMA (whose fragments were read before it), so that the
        // matrix core works through the wait; every LDS read and load of the unit follows it
        if (i == 0) {
          __builtin_amdgcn_sched_barrier(0);
          wait_barrier<WAITN, LGK>();
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if constexpr (ISSUE) {
        if (i % kEvery == kAt) issue_load<IS, PAIR>(L, ls, i / kEvery);
      }
      if constexpr (NEXT) {
        if (i % kFragStep == 0 && i / kFragStep < 4 + NY) {
          const int f = i / kFragStep;
          if (f >= 1 && f <= NY) b[Q][f - 1] = read_frag<BKC, PAIR, NJ>(nb, 32 * NY * wn + 32 * (f - 1), lane);
          else {
            const int fa = f == 0 ? 0 : f - NY;
            a[Q][fa] = read_frag<AKC, PAIR, NJ>(na, 128 * wm + 32 * fa, lane);
          }
        }
      }
    }
  }
  if constexpr (NEXT) {
    // keep the LDS reads spread over the MFMA stream: MFMA, DS read(s), MFMA, DS read(s), ...
#pragma unroll
    for (int i = 0; i < kMf; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, NY == 4 ? 1 : 2, 0);
    }
  }
}

// LDS reads one unit issues for the next (2 per K-contiguous fragment, 4 per M / N-contiguous one)
template <bool AKC, bool BKC, int NY> constexpr int kUnitReads = 4 * (AKC ? 2 : 4) + NY * (BKC ? 2 : 4);

// The K loop of one block (nk units of 64 K) with the 4-slot ring: unit s is stage s in slot s % 4
template <int AT, int BT, bool AKC, bool BKC, int NY>
__device__ __forceinline__ void k_loop(const Loads<false> &L, int nk, int lane, int wm, int wn, v8i (&a)[2][4],
                                       v8i (&b)[2][4], v16f (&acc)[4][4]) {
  constexpr int W = Ring<false>::kW1;
  // the barrier before unit s completes the reads of stage s - 1's fragments (issued during unit s - 2),
  // not all of stage s's (issued during unit s - 1): at most one unit's reads stay outstanding
  constexpr int kLgk = kUnitReads<AKC, BKC, NY> < 15 ? kUnitReads<AKC, BKC, NY> : 15;
  // stages 0..2 in flight; stage 0's fragments once it has landed
  issue_stage<0, false>(L, 0);
  issue_stage<1, false>(L, 1);
  issue_stage<2, false>(L, 2);
  wait_barrier<2 * W>();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a[0][x] = read_frag<AKC, false, 0>(lds_a<0>(), 128 * wm + 32 * x, lane);
    if (x < NY) b[0][x] = read_frag<BKC, false, 0>(lds_b<0>(), 32 * NY * wn + 32 * x, lane);
  }
  // four stages per iteration, each awaiting s + 1 (s + 2 in flight) and issuing s + 3; then the last
  // four drain the ring (nk % 4 == 0, nk >= 8)
  // the first iteration, peeled: its first unit starts the accumulators (nk >= 8)
  f8_unit<false, 0, true, W, kLgk, true, 1, 0, true, 3, AT, BT, AKC, BKC, NY, true>(L, 3, lane, wm, wn, a, b, acc);
  f8_unit<false, 1, true, W, kLgk, true, 2, 0, true, 0, AT, BT, AKC, BKC, NY>(L, 4, lane, wm, wn, a, b, acc);
  f8_unit<false, 0, true, W, kLgk, true, 3, 0, true, 1, AT, BT, AKC, BKC, NY>(L, 5, lane, wm, wn, a, b, acc);
  f8_unit<false, 1, true, W, kLgk, true, 0, 0, true, 2, AT, BT, AKC, BKC, NY>(L, 6, lane, wm, wn, a, b, acc);
  int s = 4;
  for (; s < nk - 4; s += 4) {
    f8_unit<false, 0, true, W, kLgk, true, 1, 0, true, 3, AT, BT, AKC, BKC, NY>(L, s + 3, lane, wm, wn, a, b, acc);
    f8_unit<false, 1, true, W, kLgk, true, 2, 0, true, 0, AT, BT, AKC, BKC, NY>(L, s + 4, lane, wm, wn, a, b, acc);
    f8_unit<false, 0, true, W, kLgk, true, 3, 0, true, 1, AT, BT, AKC, BKC, NY>(L, s + 5, lane, wm, wn, a, b, acc);
    f8_unit<false, 1, true, W, kLgk, true, 0, 0, true, 2, AT, BT, AKC, BKC, NY>(L, s + 6, lane, wm, wn, a, b, acc);
  }
  f8_unit<false, 0, true, W, kLgk, true, 1, 0, true, 3, AT, BT, AKC, BKC, NY>(L, s + 3, lane, wm, wn, a, b, acc);
  f8_unit<false, 1, true, W, kLgk, true, 2, 0, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<false, 0, true, 0, kLgk, true, 3, 0, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<false, 1, false, 0, 0, false, 0, 0, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
}

// The K loop with the 2-stage ring: stage p (units 2p, 2p + 1) in region p % 2
template <int AT, int BT, bool AKC, bool BKC, int NY>
__device__ __forceinline__ void k_loop(const Loads<true> &L, int nk, int lane, int wm, int wn, v8i (&a)[2][4],
                                       v8i (&b)[2][4], v16f (&acc)[4][4]) {
  constexpr int W = Ring<true>::kW1;
  const int np = nk / 2;  // stages: even, >= 4
  // stages 0 and 1 in flight; stage 0's first-unit fragments once it has landed
  issue_stage<0, true>(L, 0);
  issue_stage<1, true>(L, 1);
  wait_barrier<W>();
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a[0][x] = read_frag<AKC, true, 0>(lds_a<0>(), 128 * wm + 32 * x, lane);
    if (x < NY) b[0][x] = read_frag<BKC, true, 0>(lds_b<0>(), 32 * NY * wn + 32 * x, lane);
  }
  // two stages (one per region) per iteration, each issuing stage p + 2 in its second unit; then the
  // last two stages
  // the first iteration, peeled: its first unit starts the accumulators (np >= 4)
  f8_unit<true, 0, false, 0, 0, true, 0, 1, false, 0, AT, BT, AKC, BKC, NY, true>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<true, 1, true, 0, 0, true, 1, 0, true, 0, AT, BT, AKC, BKC, NY>(L, 2, lane, wm, wn, a, b, acc);
  f8_unit<true, 0, false, 0, 0, true, 1, 1, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<true, 1, true, 0, 0, true, 0, 0, true, 1, AT, BT, AKC, BKC, NY>(L, 3, lane, wm, wn, a, b, acc);
  int p = 2;
  for (; p < np - 2; p += 2) {
    f8_unit<true, 0, false, 0, 0, true, 0, 1, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
    f8_unit<true, 1, true, 0, 0, true, 1, 0, true, 0, AT, BT, AKC, BKC, NY>(L, p + 2, lane, wm, wn, a, b, acc);
    f8_unit<true, 0, false, 0, 0, true, 1, 1, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
    f8_unit<true, 1, true, 0, 0, true, 0, 0, true, 1, AT, BT, AKC, BKC, NY>(L, p + 3, lane, wm, wn, a, b, acc);
  }
  f8_unit<true, 0, false, 0, 0, true, 0, 1, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<true, 1, true, 0, 0, true, 1, 0, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<true, 0, false, 0, 0, true, 1, 1, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
  f8_unit<true, 1, false, 0, 0, false, 0, 0, false, 0, AT, BT, AKC, BKC, NY>(L, 0, lane, wm, wn, a, b, acc);
}

// Persistent: block b takes the launch's tiles (tile, split indices) b, b + gridDim.x, ... -- with a grid that
// is a multiple of 8, in the same XCD-aware order as one block per tile, and a tile's stores drain while the
// next tile's first stages load (8192^3: 387.5 -> 383.9 us in an A/B run; the same bits).
template <int AT, int BT, bool AKC, bool BKC, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_f8_kernel(TileArgs t0, Epilogue e0, int simple, int vec) {
  constexpr bool PAIR = BKC;  // the ring shape measured faster for this layout
  __shared__ float red[kThreads / 64];
  const int tid0 = threadIdx.x, lane0 = tid0 & 63, wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  float sa1, sb1;  // per-tensor scales: the same for every tile and split
  epilogue_scales(e0, sa1, sb1);
  float mx = 0.f;
  late_start(t0, 512ull * (t0.k / kUnitK));  // about half a tile: 16 MFMAs of 64 cycles per unit, half of them
  for (int blk = blockIdx.x; blk < t0.count; blk += gridDim.x) {
    // lane and thread ids made opaque per tile, so that nothing derived from them is hoisted out of the tile
    // loop and kept live across the K loop (that spilled 184 bytes)
    // (the wave index too: an LDS address derived from it was otherwise kept in a register across the tile
    // loop and spilled; without the spill no instance uses scratch memory, at the same speed)
    int lane = lane0, tid = tid0, wv = wave;
    asm volatile("" : "+v"(lane), "+v"(tid), "+s"(wv));
    TileArgs t = t0;
    Epilogue e = e0;
    int tm, tn, sp;
    tile_of(blk, t, tm, tn, sp);
    apply_split(t, e, sp);
    const int i0 = tm * kBM, j0 = tn * kBN;

    v16f acc[4][4];          // started by the K loop's first unit
    v8i a[2][4], b[2][4];  // fragments, double-buffered by unit parity
    const Loads<PAIR> L = make_loads<AKC, BKC, PAIR>(t, i0, j0, wv, lane);
    k_loop<AT, BT, AKC, BKC, 4>(L, t.k / kUnitK, lane, wm, wn, a, b, acc);

    mx = fmaxf(mx, tile_epilogue<EPI>(t, e, acc, i0, j0, wm, wn, lane, tid, simple, vec, sa1, sb1));
    __syncthreads();  // the write-out's ring reads are done before the next tile's loads refill the ring
  }
  if (e0.amax) amax_commit_block(e0.amax, mx, red);
}

// A launch of 256 x 128 half tiles (block b: half b % 2 of tile first + b / 2): the same K loop with 128 x 64
// per wave.  Each output's products accumulate in the same order as in a whole tile, so the results are the
// same bits.  Used for a last round of tiles at most half as large as the CU count, whose half tiles then
// fill the device.
template <int AT, int BT, bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads, 1) void gemm_f8_half_kernel(TileArgs t, Epilogue e, int vec) {
  constexpr bool PAIR = BKC;
  __shared__ float red[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn, h;
  tile_of_half(blockIdx.x, t, tm, tn, h);
  const int i0 = tm * kBM, j0 = tn * kBN + 128 * h;
  if (j0 >= t.n) return;  // the right half of a tile narrower than 129 columns: nothing to do (whole block)

  v16f acc[4][4];  // blocks y < 2 started by the K loop's first unit; the others are not used
  v8i a[2][4], b[2][4];
  const Loads<PAIR> L = make_loads<AKC, BKC, PAIR>(t, i0, j0, wave, lane);
  k_loop<AT, BT, AKC, BKC, 2>(L, t.k / kUnitK, lane, wm, wn, a, b, acc);

  __builtin_amdgcn_sched_barrier(0);
  const float mx = half_tile_epilogue(t, e, acc, i0, j0, wm, wn, lane, tid, vec);
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

// cus > 0: the grid is at most cus blocks (persistent).  tail_half (unsplit launches only): when the last
// round of tiles over cus CUs is at most half full, the whole rounds run as one launch and the last round's
// tiles as a launch of half tiles.
template <int AT, int BT, bool AKC, bool BKC>
hipError_t run_d(const TileArgs &t0, const Epilogue &e, int cus, int tail_half, hipStream_t s) {
  TileArgs t = t0;
  const int tiles = t.tiles_m * t.tiles_n;
  int whole = tiles * t.splits, tail = 0;
  if (tail_half && cus > 0 && t.splits == 1) {
    const int rounds = (tiles + cus - 1) / cus, last = tiles - (rounds - 1) * cus;
    if (2 * last <= cus) {
      whole = (rounds - 1) * cus;
      tail = last;
    }
  }
  const int grid = cus > 0 && whole > cus ? cus : whole;
  // the staged epilogues write 4-element groups of D and read OUTER scales of A as 16-byte vectors
  const int vec = ((uintptr_t)e.d % (4 * elem_bytes(e.d_dtype))) == 0 && e.ldd % 4 == 0 &&
                  (!e.sa_vec || (uintptr_t)e.sa % 16 == 0);
  const int simple = e.bias == nullptr && e.beta == 0.f && vec;
  if (whole > 0) {
    t.first = 0;
    t.count = whole;
    switch (epilogue_class(t.m, t.n, e, simple, vec)) {  // D's dtype is a run-time choice of the epilogue
      case kEpiFast16: gemm_f8_kernel<AT, BT, AKC, BKC, kEpiFast16><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
      case kEpiFull: gemm_f8_kernel<AT, BT, AKC, BKC, kEpiFull><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
      default: gemm_f8_kernel<AT, BT, AKC, BKC, kEpiAny><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
    }
  }
  if (tail > 0) {
    t.first = whole;
    t.count = tail;
    gemm_f8_half_kernel<AT, BT, AKC, BKC><<<2 * tail, kThreads, 0, s>>>(t, e, vec);
  }
  return hipGetLastError();
}

// every FP8 pairing for one layout pair; with splits > 1, k is split into equal parts and e describes
// the FP32 partial output of split 0 (the next split's follows at e.ldd * n floats)
template <bool AKC, bool BKC>
hipError_t launch_layout(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                         int k, int splits, int cus, int tail_half, const Epilogue &e, hipStream_t s) {
  const int ks = k / splits, tm = (m + kBM - 1) / kBM, tn = (n + kBN - 1) / kBN;
  const TileArgs t{A, B, lda, ldb, m, n, ks, tm, tn, splits, AKC ? ks : ks * lda, BKC ? ks : ks * ldb, e.ldd * n * 4,
                   0, tm * tn * splits};
  if (at == E5MA_E5M2)
    return bt == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_E5M2, AKC, BKC>(t, e, cus, tail_half, s)
                           : run_d<E5MA_E5M2, E5MA_E4M3, AKC, BKC>(t, e, cus, tail_half, s);
  return bt == E5MA_E5M2 ? run_d<E5MA_E4M3, E5MA_E5M2, AKC, BKC>(t, e, cus, tail_half, s)
                         : run_d<E5MA_E4M3, E5MA_E4M3, AKC, BKC>(t, e, cus, tail_half, s);
}

}  // namespace f8k
}  // namespace
}  // namespace e5ma
