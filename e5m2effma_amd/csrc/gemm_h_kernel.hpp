// gemm_h_kernel.hpp -- the fast path of e5ma_gemm on the BF16 matrix cores ("H" mode): an FP8 A times an
// FP8 B with k < kF8MinK (where the FP8 matrix cores' accumulation is not accurate enough,
// gemm_common.hpp), or times a BF16 B (FP8 weights x BF16 activations) at any k.  FP8 is widened to
// BF16 exactly (every FP8 value is a BF16 value), so every product is exact and the FP32 accumulation
// meets the contract bound.  Replaces the reference's FFMA tile loop (src/gemm_e5m2effma.cuh:117-233)
// for these cases.  Included by one translation unit per layout pair (gemm_h_tn/nn/nt/tt.hip).
//
// The block tile, ring, loads, tile order and epilogue are those of the FP8 kernel (gemm_tile.hpp).
// What differs:
// - v_mfma_f32_32x32x16_bf16: 16 k per instruction, 8 BF16 per lane and operand.
// - A stage holds KS k: 64 with an FP8 B (both operands 16 KiB), 32 with a BF16 B (A 8 KiB, B 16 KiB),
//   so that a stage is 64 resp. 32 MFMAs per wave.
// - Operands stay in their storage format in LDS (FP8 costs half the LDS traffic of BF16).  A lane
//   reads the KS / 2 consecutive k of its row that it always reads (the FP8 kernel's fragment reads),
//   and MFMA step s takes k 8 s .. 8 s + 7 of them.  Any order of the k inside a stage is a valid
//   reduction order as long as A and B use the same one, and they do.
// - FP8 fragments are widened per step with v_cvt_scalef32_pk_bf16_{fp8,bf8} (two values per
//   instruction, scale 1: exact), A once per (step, row block) and B once per (step, column block).
// LDS layouts by operand: FP8 K-contiguous, rows of KS bytes (64: chunk c at c ^ ((r >> 2) & 3); 32:
// chunk c at c ^ ((r >> 3) & 1) -- both put 16 consecutive rows' reads of one chunk on 64 distinct
// banks); BF16 K-contiguous, rows of 64 bytes (swizzle of the 64-byte rows); FP8 M / N-contiguous, KS
// k-rows of 256 bytes read with ds_read_b64_tr_b8 exactly as in the FP8 kernel.
#pragma once
#include "gemm_tile.hpp"

namespace e5ma {
namespace {
namespace hk {

using namespace tile;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kSlots = 4;

// operand geometry: dtype T, K-contiguous KC, KS k per stage
template <int T, bool KC, int KS> struct OpGeo {
  static constexpr bool kF8 = is_fp8(T);
  static constexpr int kRowBytes = KC ? (kF8 ? KS : 2 * KS) : 256;  // LDS row: a tile row, or a k-row
  static constexpr int kStageBytes = KC ? kBM * kRowBytes : KS * 256;
  static constexpr int kLoadsPerWave = kStageBytes / 1024 / 4;    // 1 KiB direct-to-LDS loads
  static constexpr int kFragDw = kF8 ? KS / 8 : KS / 4;           // dwords per lane and 32-row block
  static constexpr int kEsz = kF8 ? 1 : 2;
  static_assert(kStageBytes <= kBufBytes, "stage exceeds a ring buffer");
};

template <int RB> __device__ __forceinline__ int swz_row(int r) {
  if constexpr (RB == 64) return (r >> 2) & 3;
  else return (r >> 3) & 1;
}

// load blk (of this operand's stage) into LDS buffer lds.  K-contiguous: 1024 / RB rows of RB bytes,
// rows r0 + ... (rows past lim repeat row lim - 1, never stored).  M / N-contiguous: k-rows 4 blk .. + 3,
// 256 bytes of rows r0 .. r0 + 255 (chunks past lim, a multiple of 16, repeat the last chunk).
template <class G, bool KC>
__device__ __forceinline__ void load_op(const uint8_t *P, long long ld, int lim, int k0, int r0, int blk, int lane,
                                        uint8_t *lds) {
  if constexpr (KC) {
    constexpr int RB = G::kRowBytes, CPR = RB / 16;
    const int r = blk * (1024 / RB) + lane / CPR;
    const int c = (lane % CPR) ^ swz_row<RB>(r);
    load_lds16(P + (long long)min(r0 + r, lim - 1) * ld + (long long)k0 * G::kEsz + 16 * c, lds + blk * 1024);
  } else {
    const int kk = blk * 4 + (lane >> 4);
    const int c = (lane & 15) ^ ((kk & 7) << 1);
    load_lds16(P + (long long)(k0 + kk) * ld + min(r0 + 16 * c, lim - 16), lds + blk * 1024);
  }
}

// raw fragment of one 32-row block: lane l holds the KS / 2 k [KS / 2 * (l / 32), + KS / 2) of row
// r0 + l % 32, in storage format
template <class G, bool KC, int KS> struct Frag {
  int w[G::kFragDw];
};

// part q of a raw fragment: one 16-byte chunk of the lane's k (K-contiguous), or one transposing read of
// 8 k (M / N-contiguous)
template <class G, bool KC, int KS> constexpr int kParts = KC ? G::kFragDw / 4 : KS / 16;

template <class G, bool KC, int KS>
__device__ __forceinline__ void read_part(Frag<G, KC, KS> &f, const uint8_t *s, int r0, int lane, int q) {
  if constexpr (KC) {
    constexpr int RB = G::kRowBytes, n = G::kFragDw / 4;
    const int r = r0 + (lane & 31);
    const uint4 v = *(const uint4 *)(s + r * RB + 16 * ((n * (lane >> 5) + q) ^ swz_row<RB>(r)));
    f.w[4 * q] = (int)v.x; f.w[4 * q + 1] = (int)v.y; f.w[4 * q + 2] = (int)v.z; f.w[4 * q + 3] = (int)v.w;
  } else {
    // transposing reads, as in the FP8 kernel: this lane addresses k-row (KS / 2)(g / 2) + 8 q + b,
    // rows r .. r + 7 (r = r0 + 16 (g % 2) + 8 h); it receives row r0 + l % 32, k (KS / 2)(l / 32) + 8 q ..
    const int g = lane >> 4, h = lane & 1, b = (lane & 15) >> 1;
    const int r = r0 + 16 * (g & 1) + 8 * h;
    const uint8_t *p = s + ((KS / 2) * (g >> 1) + b) * 256 + 16 * ((r >> 4) ^ (b << 1)) + (r & 15);
    const v2i t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(p + q * 8 * 256));
    f.w[2 * q] = t.x;
    f.w[2 * q + 1] = t.y;
  }
}

template <class G, bool KC, int KS>
__device__ __forceinline__ void read_frag(Frag<G, KC, KS> &f, const uint8_t *s, int r0, int lane) {
#pragma unroll
  for (int q = 0; q < kParts<G, KC, KS>; ++q) read_part(f, s, r0, lane, q);
}

// the 8 BF16 of MFMA step s: k 8 s .. 8 s + 7 of the lane's KS / 2
template <int T, class F> __device__ __forceinline__ v8bf step_bf16(const F &f, int s) {
  if constexpr (is_fp8(T)) {
    bf16x2 p[4];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int w = f.w[2 * s + d];
      if constexpr (T == E5MA_E5M2) {
        p[2 * d] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false);
        p[2 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true);
      } else {
        p[2 * d] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
        p[2 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
      }
    }
    return __builtin_bit_cast(v8bf, v4i{__builtin_bit_cast(int, p[0]), __builtin_bit_cast(int, p[1]),
                                        __builtin_bit_cast(int, p[2]), __builtin_bit_cast(int, p[3])});
  } else {
    return __builtin_bit_cast(v8bf, v4i{f.w[4 * s], f.w[4 * s + 1], f.w[4 * s + 2], f.w[4 * s + 3]});
  }
}

template <int AT, int BT, bool AKC, bool BKC> struct Cfg {
  static constexpr int KS = BT == E5MA_BF16 ? 32 : 64;
  using GA = OpGeo<AT, AKC, KS>;
  using GB = OpGeo<BT, BKC, KS>;
  using FA = Frag<GA, AKC, KS>;
  using FB = Frag<GB, BKC, KS>;
  static constexpr int kLoads = GA::kLoadsPerWave + GB::kLoadsPerWave;  // per wave and stage
};

// part x (of 4) of this wave's loads of stage s into slot SLOT
template <class C, int SLOT, bool AKC, bool BKC>
__device__ __forceinline__ void issue_part(const TileArgs &t, int s, int i0, int j0, int wave, int lane, int x) {
#pragma unroll
  for (int q = 0; q < C::GA::kLoadsPerWave; ++q)
    if (q % 4 == x) load_op<typename C::GA, AKC>(t.A, t.lda, t.m, s * C::KS, i0, wave * C::GA::kLoadsPerWave + q, lane,
                                                  lds_a<SLOT>());
#pragma unroll
  for (int q = 0; q < C::GB::kLoadsPerWave; ++q)
    if (q % 4 == x) load_op<typename C::GB, BKC>(t.B, t.ldb, t.n, s * C::KS, j0, wave * C::GB::kLoadsPerWave + q, lane,
                                                  lds_b<SLOT>());
}

// Stage s (= SLOT mod 4) of the K loop; a / b hold stage s's raw fragments.  WAITN, NEXT, ISSUE as in the
// FP8 kernel.  Steps outer: B's four column blocks are widened once per step, A's row block once per
// (step, x).  Raw fragments are refilled from stage s + 1 once this stage no longer needs them:
// - FP8 x FP8: each fragment in the last step, right after it was widened, the LDS reads spread over
//   that step's MFMAs;
// - BF16 B: its fragments are the MFMA operands themselves, so a whole-stage refill could only follow
//   the stage's last MFMAs, and the next stage's first MFMAs would wait for it.  Each part is refilled
//   after the MFMAs of the step that uses it, so the reads of stage s + 1 spread over the stage (E5M2 x
//   BF16, A / B on two boxes: 8192^3 TN -1.7 to -2.0 %, 8192^2 x 4096 NN -1.5 to -2.7 %); A as for FP8 x
//   FP8.  The same order for FP8 x FP8 measured 1 % slower.
// The loads of stage s + 4 go out during step 0.
template <class C, int WAITN, bool NEXT, bool ISSUE, int SLOT, int AT, int BT, bool AKC, bool BKC>
__device__ __forceinline__ void h_stage(const TileArgs &t, int s, int i0, int j0, int wave, int lane, int wm, int wn,
                                        typename C::FA (&a)[4], typename C::FB (&b)[4], v16f (&acc)[4][4]) {
  constexpr int S = C::KS / 16;
  constexpr bool kPerStep = !is_fp8(BT);
  if constexpr (NEXT) wait_barrier<WAITN>();
  const uint8_t *na = lds_a<(SLOT + 1) & 3>(), *nb = lds_b<(SLOT + 1) & 3>();
#pragma unroll
  for (int st = 0; st < S; ++st) {
    v8bf bb[4];
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      bb[y] = step_bf16<BT>(b[y], st);
      if constexpr (NEXT && !kPerStep) {
        if (st == S - 1) read_frag(b[y], nb, 128 * wn + 32 * y, lane);
      }
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const v8bf aa = step_bf16<AT>(a[x], st);
      if constexpr (NEXT) {
        if (st == S - 1) read_frag(a[x], na, 128 * wm + 32 * x, lane);
      }
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aa, bb[y], acc[x][y], 0, 0, 0);
        if constexpr (ISSUE) {
          if (st == 0 && y == 1) issue_part<C, SLOT, AKC, BKC>(t, s + 4, i0, j0, wave, lane, x);
        }
      }
    }
    if constexpr (kPerStep) {
      if constexpr (NEXT) {
#pragma unroll
        for (int y = 0; y < 4; ++y) read_part(b[y], nb, 128 * wn + 32 * y, lane, st);  // BF16: part st = step st
      }
      __builtin_amdgcn_sched_barrier(0);  // each step's reads stay in that step
    }
  }
}

template <int AT, int BT, bool AKC, bool BKC, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_h_kernel(TileArgs t0, Epilogue e0, int simple, int vec) {
  using C = Cfg<AT, BT, AKC, BKC>;
  __shared__ float red[kThreads / 64];
  const int tid0 = threadIdx.x, lane0 = tid0 & 63, wave0 = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int wm = wave0 >> 1, wn = wave0 & 1;
  float sa1, sb1;  // per-tensor scales: the same for every tile and split
  epilogue_scales(e0, sa1, sb1);
  float mx = 0.f;
  // a stage is KS k of 16 MFMAs of 32 cycles per 16 k per wave: about half a tile is 256 cycles per k-step
  late_start(t0, 256ull * (t0.k / 16));
  for (int blk = blockIdx.x; blk < t0.count; blk += gridDim.x) {
    // lane and thread ids made opaque per tile, so that nothing derived from them is hoisted out of the tile loop
    // (the wave index too: values derived from it were otherwise kept in registers across the tile loop and
    // spilled, 32 registers in the full-tile write-out's instances; none uses scratch memory now)
    int lane = lane0, tid = tid0, wave = wave0;
    asm volatile("" : "+v"(lane), "+v"(tid), "+s"(wave));
    TileArgs t = t0;
    Epilogue e = e0;
    int tm, tn, sp;
    tile_of(blk, t, tm, tn, sp);
    apply_split(t, e, sp);
    const int i0 = tm * kBM, j0 = tn * kBN;
    const int nk = t.k / C::KS;

    v16f acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

    // prologue: stages 0..2 in flight; stage 3 is issued once every wave is past the first barrier
#pragma unroll
    for (int x = 0; x < 4; ++x) issue_part<C, 0, AKC, BKC>(t, 0, i0, j0, wave, lane, x);
#pragma unroll
    for (int x = 0; x < 4; ++x) issue_part<C, 1, AKC, BKC>(t, 1, i0, j0, wave, lane, x);
#pragma unroll
    for (int x = 0; x < 4; ++x) issue_part<C, 2, AKC, BKC>(t, 2, i0, j0, wave, lane, x);
    wait_barrier<2 * C::kLoads>();  // stage 0 landed; stages 1 and 2 may be in flight
#pragma unroll
    for (int x = 0; x < 4; ++x) issue_part<C, 3, AKC, BKC>(t, 3, i0, j0, wave, lane, x);
    typename C::FA a[4];
    typename C::FB b[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      read_frag(a[x], lds_a<0>(), 128 * wm + 32 * x, lane);
      read_frag(b[x], lds_b<0>(), 128 * wn + 32 * x, lane);
    }
    constexpr int kW2 = 2 * C::kLoads, kW1 = C::kLoads;
    int s = 0;
    for (; s < nk - 4; s += 4) {
      h_stage<C, kW2, true, true, 0, AT, BT, AKC, BKC>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
      h_stage<C, kW2, true, true, 1, AT, BT, AKC, BKC>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
      h_stage<C, kW2, true, true, 2, AT, BT, AKC, BKC>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
      h_stage<C, kW2, true, true, 3, AT, BT, AKC, BKC>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);
    }
    h_stage<C, kW2, true, false, 0, AT, BT, AKC, BKC>(t, s, i0, j0, wave, lane, wm, wn, a, b, acc);
    h_stage<C, kW1, true, false, 1, AT, BT, AKC, BKC>(t, s + 1, i0, j0, wave, lane, wm, wn, a, b, acc);
    h_stage<C, 0, true, false, 2, AT, BT, AKC, BKC>(t, s + 2, i0, j0, wave, lane, wm, wn, a, b, acc);
    h_stage<C, 0, false, false, 3, AT, BT, AKC, BKC>(t, s + 3, i0, j0, wave, lane, wm, wn, a, b, acc);

    mx = fmaxf(mx, tile_epilogue<EPI>(t, e, acc, i0, j0, wm, wn, lane, tid, simple, vec, sa1, sb1));
    __syncthreads();  // the write-out's ring reads are done before the next tile's loads refill the ring
  }
  if (e0.amax) amax_commit_block(e0.amax, mx, red);
}

template <int AT, int BT, bool AKC, bool BKC>
hipError_t run_d(const TileArgs &t, const Epilogue &e, int cus, hipStream_t s) {
  // persistent: at most one block per CU (cus > 0), each looping over its tiles in the XCD-aware order
  const int whole = t.tiles_m * t.tiles_n * t.splits, grid = cus > 0 && whole > cus ? cus : whole;
  const int vec = ((uintptr_t)e.d % (4 * elem_bytes(e.d_dtype))) == 0 && e.ldd % 4 == 0 &&
                  (!e.sa_vec || (uintptr_t)e.sa % 16 == 0);
  const int simple = e.bias == nullptr && e.beta == 0.f && vec;
  switch (epilogue_class(t.m, t.n, e, simple, vec)) {  // D's dtype is a run-time choice of the epilogue
    case kEpiFast16: gemm_h_kernel<AT, BT, AKC, BKC, kEpiFast16><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
    case kEpiFull: gemm_h_kernel<AT, BT, AKC, BKC, kEpiFull><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
    default: gemm_h_kernel<AT, BT, AKC, BKC, kEpiAny><<<grid, kThreads, 0, s>>>(t, e, simple, vec); break;
  }
  return hipGetLastError();
}

// the FP8 A x FP8 B pairings for one layout pair (lda / ldb in elements; splits as in the FP8 kernel)
template <bool AKC, bool BKC>
hipError_t launch_layout(int at, int bt, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m, int n,
                         int k, int splits, int cus, const Epilogue &e, hipStream_t s) {
  const int ks = k / splits;
  const int tm = (m + kBM - 1) / kBM, tn = (n + kBN - 1) / kBN;
  const TileArgs t{A, B, lda, ldb, m, n, ks, tm, tn, splits, AKC ? ks : ks * lda, BKC ? ks : ks * ldb, e.ldd * n * 4,
                   0, tm * tn * splits};
  if (at == E5MA_E5M2)
    return bt == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_E5M2, AKC, BKC>(t, e, cus, s)
                           : run_d<E5MA_E5M2, E5MA_E4M3, AKC, BKC>(t, e, cus, s);
  return bt == E5MA_E5M2 ? run_d<E5MA_E4M3, E5MA_E5M2, AKC, BKC>(t, e, cus, s)
                         : run_d<E5MA_E4M3, E5MA_E4M3, AKC, BKC>(t, e, cus, s);
}

// FP8 A x K-contiguous BF16 B (ldb in elements)
template <bool AKC>
hipError_t launch_layout_bf16(int at, int, const uint8_t *A, long long lda, const uint8_t *B, long long ldb, int m,
                              int n, int k, int splits, int cus, const Epilogue &e, hipStream_t s) {
  const int ks = k / splits;
  const int tm = (m + kBM - 1) / kBM, tn = (n + kBN - 1) / kBN;
  const TileArgs t{A, B, lda, 2 * ldb, m, n, ks, tm, tn, splits, AKC ? ks : ks * lda, 2LL * ks, e.ldd * n * 4,
                   0, tm * tn * splits};
  return at == E5MA_E5M2 ? run_d<E5MA_E5M2, E5MA_BF16, AKC, true>(t, e, cus, s)
                         : run_d<E5MA_E4M3, E5MA_BF16, AKC, true>(t, e, cus, s);
}

}  // namespace hk
}  // namespace
}  // namespace e5ma
