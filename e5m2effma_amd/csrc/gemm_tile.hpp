// gemm_tile.hpp -- what the matrix-core tile kernels (gemm_f8_kernel.hpp, gemm_h_kernel.hpp) share:
// the 256 x 256 block tile of 4 waves (128 x 128 accumulators each, 4 x 4 blocks of 32 x 32), the
// 128 KiB LDS ring of 8 buffers and its direct-to-LDS loads, the XCD-aware tile order, and the
// epilogues, which stage the finished tile in the ring.
#pragma once
#include <type_traits>

#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {
namespace {
namespace tile {

using namespace dev;
using namespace gemm;

constexpr int kBM = 256, kBN = 256, kThreads = 256;
constexpr int kBufBytes = 16384;  // one ring buffer (an operand stage of up to 16 KiB)
constexpr int kGroupM = 4;        // tile order: groups of 4 m-tiles

typedef __attribute__((address_space(3))) v2i lds_v2i;

// The LDS ring: 128 KiB as two 32 KiB regions per operand, each its own object.  The FP8 kernel uses
// each region as one 128-byte K stage of an operand; the BF16-matrix-core kernel and the epilogue use
// the 8 halves (16 KiB buffers: 4 slots x 2 operands, or 8 column groups) with compile-time indices.
__shared__ __attribute__((aligned(1024))) uint8_t g_ra0[2 * kBufBytes], g_ra1[2 * kBufBytes];
__shared__ __attribute__((aligned(1024))) uint8_t g_rb0[2 * kBufBytes], g_rb1[2 * kBufBytes];
template <int S> __device__ __forceinline__ uint8_t *lds_a() { return (S < 2 ? g_ra0 : g_ra1) + (S & 1) * kBufBytes; }
template <int S> __device__ __forceinline__ uint8_t *lds_b() { return (S < 2 ? g_rb0 : g_rb1) + (S & 1) * kBufBytes; }
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

// One accumulator element copied to a VGPR where it is used.  The "a" constraint keeps the value in
// its accumulator register; left to itself the compiler copies whole accumulator blocks to VGPRs at
// the end of the K loop and spills them.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// s_waitcnt vmcnt(N) lgkmcnt(LGK), then s_barrier; the memory clobber keeps the compiler from moving
// memory operations across it.  (__syncthreads would also wait for every outstanding global load.)
// LDS reads complete in issue order, so lgkmcnt(LGK) leaves at most the LGK latest reads (and scalar
// loads) in flight.
template <int N, int LGK = 0> __device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(%1)\n\ts_barrier" ::"n"(N), "n"(LGK) : "memory");
}

struct TileArgs {
  const uint8_t *A, *B;
  long long lda, ldb;  // in bytes
  int m, n, k;         // k: the K range of one block (of one split)
  int tiles_m, tiles_n;
  int splits;                 // K splits (1: none); split s writes FP32 partials at D + s * d_split
  long long a_split, b_split;  // bytes from one split's first A / B element to the next split's
  long long d_split;          // bytes between the splits' partial outputs
  int first, count;           // this launch's (tile, split) indices: first .. first + count - 1
};

// Output tile and K split of block b.  XCD-aware when the block count is a multiple of 8 (blocks are
// dispatched to the 8 XCDs round-robin): an XCD runs consecutive indices x, so with K splits each XCD
// works on one split (one K slice of the operands in its L2); then tiles are grouped kGroupM m-tiles
// at a time.
__device__ __forceinline__ void tile_of(int b, const TileArgs &t, int &tm, int &tn, int &split) {
  int tiles = t.tiles_m * t.tiles_n, per_group = kGroupM * t.tiles_n;
  // opaque per call: a persistent kernel then divides afresh per tile instead of keeping the divisions'
  // reciprocals live across its tile loop (they were spilled to scratch; the time was the same either way)
  asm volatile("" : "+s"(tiles), "+s"(per_group));
  const int total = t.count;
  int x = b;
  if ((total & 7) == 0) x = (b & 7) * (total >> 3) + (b >> 3);
  x += t.first;
  split = x / tiles;
  x -= split * tiles;
  const int g = x / per_group, r = x - g * per_group;
  const int gm = min(kGroupM, t.tiles_m - g * kGroupM);
  tm = g * kGroupM + r % gm;
  tn = r / gm;
}

// Half tile of block b of a launch of 256 x 128 half tiles (no K splits) over tiles first .. first + count - 1
// in the same (m-grouped) order.  XCD-aware like tile_of when count is a multiple of 8: XCD b % 8 runs a
// contiguous run of count / 8 tiles, both halves of each (half = index within the XCD % 2), so the tiles an
// XCD runs at once share operand slices in its L2.
__device__ __forceinline__ void tile_of_half(int b, const TileArgs &t, int &tm, int &tn, int &h) {
  int q = b;  // position among the 2 count half tiles
  if ((t.count & 7) == 0) q = (b & 7) * (t.count >> 2) + (b >> 3);
  const int x = t.first + (q >> 1);
  h = q & 1;
  const int per_group = kGroupM * t.tiles_n;
  const int g = x / per_group, r = x - g * per_group;
  const int gm = min(kGroupM, t.tiles_m - g * kGroupM);
  tm = g * kGroupM + r % gm;
  tn = r / gm;
}

// the operands and output of K split s
__device__ __forceinline__ void apply_split(TileArgs &t, Epilogue &e, int s) {
  if (s == 0) return;
  t.A += s * t.a_split;
  t.B += s * t.b_split;
  e.d = (uint8_t *)e.d + s * t.d_split;
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

// LDS byte address of p (a pointer into one of the ring buffers)
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// p (wave-uniform) in scalar registers.  Values derived from the block index can be computed in vector
// registers (integer division is), and an "s" asm operand is not moved to scalar registers by itself.
__device__ __forceinline__ const uint8_t *uniform_ptr(const uint8_t *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// The same load with a wave-uniform 64-bit base in scalar registers and a 32-bit per-lane offset
// (global_load_lds_dwordx4's saddr form: address = base + off); lds is the LDS byte address.  A loop
// that keeps each lane's offsets fixed and advances only the base issues no vector address arithmetic.
// Both scalar operands go through uniform_ptr / readfirstlane (a no-op for values already in scalar
// registers), since register pressure can leave a hoisted uniform value in a vector register.
__device__ __forceinline__ void load_lds16s(const uint8_t *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

// Four consecutive elements of dtype T at element idx (4-element aligned) as FP32 (FP8 times sinv; the
// others exact): one vector load
template <int T> __device__ __forceinline__ void load4_t(const void *p, size_t idx, float sinv, float (&o)[4]) {
  const uint8_t *b = (const uint8_t *)p + idx * elem_bytes(T);
  if constexpr (T == E5MA_FP32) {
    const float4 v = *(const float4 *)b;
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else if constexpr (elem_bytes(T) == 2) {
    const uint2 v = *(const uint2 *)b;
    const uint32_t h[4] = {v.x & 0xFFFFu, v.x >> 16, v.y & 0xFFFFu, v.y >> 16};
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = T == E5MA_BF16 ? bf16_value(h[q]) : f16_value(h[q]);
  } else {
    const uint32_t v = *(const uint32_t *)b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t c = (v >> (8 * q)) & 0xFFu;
      o[q] = (T == E5MA_E5M2 ? e5m2_value(c) : e4m3_value(c)) * sinv;
    }
  }
}
// the same with the dtype chosen at run time (one dispatch per four elements)
__device__ __forceinline__ void load4_any(int t, const void *p, size_t idx, float sinv, float (&o)[4]) {
  switch (t) {
    case E5MA_E5M2: load4_t<E5MA_E5M2>(p, idx, sinv, o); break;
    case E5MA_E4M3: load4_t<E5MA_E4M3>(p, idx, sinv, o); break;
    case E5MA_BF16: load4_t<E5MA_BF16>(p, idx, sinv, o); break;
    case E5MA_FP16: load4_t<E5MA_FP16>(p, idx, sinv, o); break;
    default: load4_t<E5MA_FP32>(p, idx, sinv, o); break;
  }
}

// Writes out one staged half tile (256 rows x 128 columns starting at column jh) in the reference's
// epilogue order (include/e5m2effma.h: v = acc * (alpha * sa[i]) * sb[j]; v += bias[i];
// v = fma(beta, C * csinv, v); amax; convert).  Wave w takes columns w, w + 4, ..., thread t rows
// i .. i + 3 (i = i0 + 4 (t % 64)); eight columns per step, with their C values loaded (one vector load
// per column when C is aligned) before any is computed or stored, so 32 values per thread are in
// flight (C may alias D: each element is read before it is written, by the same thread).  CT: the
// dtype of C, or -1 when beta = 0.
// C's / D's dtype chosen at run time, element by element (the common pairings have their own instances)
constexpr int kAnyC = 100, kAnyD = 101;

template <int DT, int CT>
__device__ __forceinline__ float general_half(const Epilogue &e, const EpiState &st, const TileArgs &t, int i, int jh,
                                              const float (&rs)[4], const float (&rb)[4], int vec, int tid,
                                              float mx) {
  constexpr int kCols = 8;  // columns per step
  const int w = tid >> 6, il = 4 * (tid & 63);
  const bool rows4 = i + 3 < t.m;
  bool cvec = false;
  if constexpr (CT == kAnyC)
    cvec = rows4 && e.beta != 0.f && (uintptr_t)e.c % (4 * elem_bytes(e.c_dtype)) == 0 && e.ldc % 4 == 0;
  else if constexpr (CT >= 0)
    cvec = rows4 && (uintptr_t)e.c % (4 * elem_bytes(CT)) == 0 && e.ldc % 4 == 0;
  const float sb1 = scale_or_one(e.sb);
#pragma unroll 1
  for (int c0 = 0; c0 < 32; c0 += kCols) {
    float a[kCols][4], cv[kCols][4];
#pragma unroll
    for (int u = 0; u < kCols; ++u) {
      const int jl = w + 4 * (c0 + u), j = jh + jl;
      const float4 v4 = *(const float4 *)(stage_at(jl >> 4) + (jl & 15) * kBM + il);
      a[u][0] = v4.x; a[u][1] = v4.y; a[u][2] = v4.z; a[u][3] = v4.w;
#pragma unroll
      for (int q = 0; q < 4; ++q) cv[u][q] = 0.f;
      if constexpr (CT == kAnyC) {
        if (j < t.n && e.beta != 0.f) {  // beta = 0: there is no C (NULL), and none is read
          if (cvec) {
            load4_any(e.c_dtype, e.c, (size_t)j * e.ldc + i, st.csinv, cv[u]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (i + q < t.m) cv[u][q] = load_any(e.c_dtype, e.c, (size_t)j * e.ldc + i + q, st.csinv);
          }
        }
      } else if constexpr (CT >= 0) {
        if (j < t.n) {
          if (cvec) {
            load4_t<CT>(e.c, (size_t)j * e.ldc + i, st.csinv, cv[u]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (i + q < t.m) cv[u][q] = load_t<CT>(e.c, (size_t)j * e.ldc + i + q, st.csinv);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kCols; ++u) {
      const int j = jh + w + 4 * (c0 + u);
      if (j >= t.n) continue;
      const float sbj = e.sb_vec ? e.sb[j] : sb1;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = a[u][q] * ((e.sa_vec || e.sb_vec) ? rs[q] * sbj : st.s);
        if (e.bias) v[q] = v[q] + rb[q];
        if constexpr (CT == kAnyC) {
          if (e.beta != 0.f) v[q] = __builtin_fmaf(e.beta, cv[u][q], v[q]);
        } else if constexpr (CT != -1) {
          v[q] = __builtin_fmaf(e.beta, cv[u][q], v[q]);
        }
      }
      const size_t o = (size_t)j * e.ldd + i;
      if constexpr (DT == kAnyD) {
        if (rows4 && vec) {
          store4_any(e.d_dtype, e.d, o, v, st.qscale);
#pragma unroll
          for (int q = 0; q < 4; ++q) mx = amax_fold(mx, v[q]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (i + q < t.m) {
              store_any(e.d_dtype, e.d, o + q, v[q], st.qscale);
              mx = amax_fold(mx, v[q]);
            }
        }
        continue;
      } else if (rows4 && vec) {
        uint8_t *dp = (uint8_t *)e.d + o * elem_bytes(DT);
        if constexpr (DT == E5MA_FP32) {
          *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
        } else if constexpr (is_fp8(DT)) {
          *(uint32_t *)dp = f32x4_to_fp8<DT>(v[0] * st.qscale, v[1] * st.qscale, v[2] * st.qscale, v[3] * st.qscale);
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

// alpha * sa and sb as per-tensor values (1 where absent or a vector), read with scalar loads when the
// kernel starts so that their latency hides behind the K loop
__device__ __forceinline__ void epilogue_scales(const Epilogue &e, float &sa1, float &sb1) {
  typedef const __attribute__((address_space(4))) float *scalar_ptr;
  sa1 = e.alpha * (e.sa && !e.sa_vec ? *(scalar_ptr)e.sa : 1.f);
  sb1 = e.sb && !e.sb_vec ? *(scalar_ptr)e.sb : 1.f;
}

// ---- epilogues of full tiles: staged through the LDS ring ----------------------------------------
// Straight from the accumulators each lane holds 4 consecutive rows of one column per block and group,
// so a store instruction would write 8-16 bytes into each of 32 columns.  Staging the tile in the ring
// (free once the K loop's last fragments are read) lets every store instruction write whole columns:
// 8 full 128-byte lines.  Measured on the 8192^3 headline (one block per CU): 21.7K cycles of epilogue
// per tile with the direct stores, 12.6K staged.
//
// Lane layout of an accumulator block (x, y) of wave (wm, wn): lane l, register 4 g + q holds output
//   i = 128 wm + 32 x + 8 g + 4 (l / 32) + q,  j = 128 wn + 32 y + l % 32   (tile coordinates).

// Every NaN among the pairs' BF16 codes becomes 0x7FC0 (include/e5m2effma.h; reference rne_hi)
__device__ __forceinline__ uint32_t bf16_pair_canonical(uint32_t w) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t v = (w >> (16 * h)) & 0xFFFFu;
    if ((v & 0x7FFFu) > 0x7F80u) w = (w & ~(0xFFFFu << (16 * h))) | (0x7FC0u << (16 * h));
  }
  return w;
}

// Set by any lane of the block whose converted values include a NaN (staged16)
__shared__ int g_nan_flag;

// BF16 output, no bias, beta = 0, no amax.  sa1 = alpha * sa, sb1 = sb (per-tensor values, read before
// the K loop); VS: row / column scale vectors (either or both).  Each (EDGE, VS) pair is its own
// straight-line copy: a copy with run-time flags held 256 VGPRs, spilled, and its scratch reload made
// every tile wait for its own stores.
// Phase W: v = acc * ((alpha * sa[i]) * sb[j]) converted to BF16; lanes l and l + 32 hold rows 8g..8g+3
// and 8g+4..8g+7 of one column, and one v_permlane32_swap per dword (which exchanges lanes 32..63 of its
// first operand with lanes 0..31 of its second) pairs groups 2p and 2p + 1 so that lane l holds rows
// 16p..16p+7 and lane l + 32 rows 16p+8..16p+15: 16 bytes each, written to column j of the ring (512 bytes;
// 32 columns per 16 KiB buffer) at 16-byte chunk k ^ (j % 16), so that the 16 lanes a ds_*_b128 serves per
// cycle meet 16 distinct bank groups.  The hardware pair conversion keeps a NaN's sign and payload: every
// lane folds 0 * v of the converted pairs into a screen that is NaN exactly when some value is NaN or Inf
// (BF16 keeps both), and a block-wide flag then makes phase R rewrite NaN codes to 0x7FC0 (rare path).
// Phase R: step q writes tile columns 8q .. 8q + 7, thread t column 8q + t / 32, rows 8 (t % 32) .. + 7.
// Full tiles read the ring 8 steps at a time before their stores, so that the LDS latency is paid once per
// 8 stores rather than once per store; edge tiles read per store (their reads sink into the store's
// predicate).
// EDGE: the tile may reach past m or n (stores and scale reads limited to D; m % 8 == 0, so a thread's 8
// rows lie all inside or all outside D).
template <bool EDGE, bool FIX>
__device__ __forceinline__ void staged16_out(const Epilogue &e, int i0, int j0, int m, int n, int tid) {
  constexpr int kBatch = EDGE ? 1 : 8;
  const int cq = tid >> 5, k = tid & 31;
  const bool rowv = i0 + 8 * k < m;
  uint8_t *gp = (uint8_t *)e.d + ((size_t)(j0 + cq) * e.ldd + i0 + 8 * k) * 2;
  const size_t gstep = (size_t)16 * e.ldd;  // 8 columns
#pragma unroll
  for (int q0 = 0; q0 < 32; q0 += kBatch) {
    uint4 d[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int q = q0 + u, cl = 8 * (q & 3) + cq;  // column within ring buffer q / 4
      d[u] = *(const uint4 *)((const uint8_t *)stage_at(q >> 2) + cl * 512 + ((k ^ (cl & 15)) << 4));
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int q = q0 + u;
      if constexpr (FIX) {
        d[u].x = bf16_pair_canonical(d[u].x); d[u].y = bf16_pair_canonical(d[u].y);
        d[u].z = bf16_pair_canonical(d[u].z); d[u].w = bf16_pair_canonical(d[u].w);
      }
      if (!EDGE || (rowv && j0 + 8 * q + cq < n)) *(uint4 *)(gp + q * gstep) = d[u];
    }
  }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <bool EDGE, bool VS>
__device__ __forceinline__ void staged16(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int m, int n, int wm,
                                         int wn, int lane, int tid, float sa1, float sb1) {
  const float s = sa1 * sb1;
  const int lc = lane & 31, hi = lane >> 5;
  float screen[2] = {0.f, 0.f};
  // VS: this lane's 4 column scales and 16 row-group scales (alpha * sa[i]), loaded together
  float sbv[4];
  float4 sav[4][4];
  if constexpr (VS) {
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int jc = j0 + 128 * wn + 32 * y + lc;  // past n (edge tiles) never stored
      sbv[y] = e.sb_vec ? e.sb[EDGE ? min(jc, n - 1) : jc] : sb1;
    }
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r4 = i0 + 128 * wm + 32 * x + 8 * g + 4 * hi;  // rows r4 .. r4 + 3
        if (e.sa_vec) {
          // rows past m (edge tiles) read the last in-range group: never stored
          const float4 a4 = *(const float4 *)(e.sa + (EDGE ? min(r4, m - 4) : r4));
          sav[x][g] = make_float4(e.alpha * a4.x, e.alpha * a4.y, e.alpha * a4.z, e.alpha * a4.w);
        } else {
          sav[x][g] = make_float4(sa1, sa1, sa1, sa1);
        }
      }
  }
  // this lane's byte offsets in a column group for register groups (x, p): column lc's 512 bytes, 16-byte
  // chunk (16 wm + 4 x + 2 p + hi) ^ (lc % 16)
  uint32_t off[4][2];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int p = 0; p < 2; ++p) off[x][p] = lc * 512 + (((16 * wm + 4 * x + 2 * p + hi) ^ (lc & 15)) << 4);
  if (tid == 0) g_nan_flag = 0;
  __syncthreads();  // every wave has read its last fragments from the ring
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    uint8_t *col = (uint8_t *)stage_at(4 * wn + y);
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        __builtin_amdgcn_sched_barrier(0);
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = 2 * p + h;
          float v[4];
          if constexpr (VS) {
            const float as[4] = {sav[x][g].x, sav[x][g].y, sav[x][g].z, sav[x][g].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * (as[q] * sbv[y]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * s;
          }
          const bf16x2 lo{(__bf16)v[0], (__bf16)v[1]}, hi2{(__bf16)v[2], (__bf16)v[3]};
          // 0 * a + 0 * b + screen per BF16 pair: NaN exactly when a or b is NaN or Inf (one instruction for
          // two values)
          screen[0] = __builtin_amdgcn_fdot2_f32_bf16(lo, bf16x2{}, screen[0], false);
          screen[1] = __builtin_amdgcn_fdot2_f32_bf16(hi2, bf16x2{}, screen[1], false);
          w[2 * h] = __builtin_bit_cast(uint32_t, lo);
          w[2 * h + 1] = __builtin_bit_cast(uint32_t, hi2);
        }
        // (w0, w1): rows 8(2p) + 4 hi .. + 3; (w2, w3): rows 8(2p + 1) + 4 hi .. + 3
        const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        *(uint4 *)(col + off[x][p]) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
      }
  }
  if (__builtin_isnan(screen[0] + screen[1])) g_nan_flag = 1;
  __syncthreads();
  if (g_nan_flag != 0) staged16_out<EDGE, true>(e, i0, j0, m, n, tid);
  else staged16_out<EDGE, false>(e, i0, j0, m, n, tid);
}

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// load4_t with non-temporal loads (C of the full-tile write-out: read once, kept out of the caches' way)
template <int T> __device__ __forceinline__ void load4_nt(const void *p, size_t idx, float sinv, float (&o)[4]) {
  const uint8_t *b = (const uint8_t *)p + idx * elem_bytes(T);
  if constexpr (T == E5MA_FP32) {
    const v4f v = __builtin_nontemporal_load((const v4f *)b);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else if constexpr (elem_bytes(T) == 2) {
    const v2u v = __builtin_nontemporal_load((const v2u *)b);
    const uint32_t h[4] = {v.x & 0xFFFFu, v.x >> 16, v.y & 0xFFFFu, v.y >> 16};
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = T == E5MA_BF16 ? bf16_value(h[q]) : f16_value(h[q]);
  } else {
    const uint32_t v = __builtin_nontemporal_load((const uint32_t *)b);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t c = (v >> (8 * q)) & 0xFFu;
      o[q] = (T == E5MA_E5M2 ? e5m2_value(c) : e4m3_value(c)) * sinv;
    }
  }
}

// Tile column of pass column pc (0..127) in pass h of staged_general: a pass takes 64 columns of each wave
// column wn = pc / 64, i.e. tile columns 128 (pc / 64) + 64 h + pc % 64.
__device__ __forceinline__ int pass_col(int h, int pc) { return 128 * (pc >> 6) + 64 * h + (pc & 63); }

// Full tile, any output dtype, bias and beta * C (CT: C's dtype, -1 when beta = 0), 4-element aligned
// D and C: two passes, each over half of the tile's columns (128 columns x 256 rows of FP32, the whole
// ring): pass h takes accumulator blocks y = 2h, 2h + 1 of every wave, so all four waves stage in each
// pass (with the halves of the tile per pass, two waves stood idle through each staging: 8.4K cycles
// per pass in TE wgrad, against its 15K-cycle write-out).
// Phase W: every wave writes v = acc * ((alpha * sa[i]) * sb[j]), 4 rows (16 bytes) per lane and group,
// pass column c at 1 KiB in buffer c / 16, 16-byte chunk k at k ^ (c % 16).
// Phase R: thread t takes rows 4 (t % 64) .. + 3 of pass column 4q + t / 64 (q = 0..31), so C is
// read and D written along whole columns; v = v + bias[i]; v = fma(beta, C * csinv, v); amax; convert
// (the order of include/e5m2effma.h).  C is loaded a group of 8 steps ahead of its use, the next half's
// first group before that half is staged (a load waited on right away left the TE wgrad GEMM 17% slower).
// C is read and D written non-temporally: an FP32 C and D (TE wgrad's main_grad, 235 MB) otherwise pushed the
// operands out of the Infinity Cache, and the K loops waited on HBM (wgrad 4096 x 14336 x 8192: 474 -> 419 us;
// either one alone: 474 / 462 us).
// C may alias D: each thread reads its own elements before it writes them, and no other thread writes them.
template <int DT, int CT, bool EDGE>
__device__ __forceinline__ float staged_general(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int m, int n,
                                                int wm, int wn, int lane, int tid, float sa1, float sb1) {
  float mx = 0.f;
  const float s = sa1 * sb1;
  const bool vs = e.sa_vec || e.sb_vec;
  const int lc = lane & 15, hi = lane >> 5, kr = tid & 63, cq = tid >> 6;
  const int i = i0 + 4 * kr;  // phase R rows i .. i + 3: all below m or none (m % 4 == 0, class precondition)
  const bool rowv = i < m;
  float rb[4] = {0.f, 0.f, 0.f, 0.f};
  if (e.bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r) rb[r] = load_any(e.bias_dtype, e.bias, (size_t)(EDGE ? min(i + r, m - 1) : i + r), 1.f);
  }
  const float csinv = scale_or_one(e.c_sinv), qs = scale_or_one(e.d_scale);
  const bool amax = e.amax != nullptr;
  // C of one group of 8 write-out steps per buffer (group g: half g / 4, steps 8 (g % 4) .. + 7), loaded one
  // group ahead of its use so that a load's latency overlaps the previous group's stores
  float ca[8][4], cb[8][4];
  auto load_group = [&](int g, float (&c)[8][4]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = 8 * (g & 3) + u;
      const int j = j0 + pass_col(g >> 2, 4 * q + cq);
#pragma unroll
      for (int r = 0; r < 4; ++r) c[u][r] = 0.f;
      // C exists for these elements (edge tiles: not past m or n); 4-element aligned (class precondition)
      if ((!EDGE || (j < n && rowv)) && (CT != kAnyC || e.beta != 0.f)) {
        if constexpr (CT == kAnyC) load4_any(e.c_dtype, e.c, (size_t)j * e.ldc + i, csinv, c[u]);
        else if constexpr (CT >= 0) load4_nt<CT>(e.c, (size_t)j * e.ldc + i, csinv, c[u]);
      }
    }
  };
  // group g's write-out with C of the group in cur, loading group g + 1's into nxt
  auto write_group = [&](int h, int gq, float (&cur)[8][4], float (&nxt)[8][4]) {
    const int g = 4 * h + gq;
    if constexpr (CT != -1) {
      if (g < 7) load_group(g + 1, nxt);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = 8 * gq + u;
      const int cl = 4 * (q & 3) + cq;  // column within ring buffer q / 4
      const int j = j0 + pass_col(h, 4 * q + cq);
      const float4 x4 = *(const float4 *)(stage_at(q >> 2) + cl * 256 + ((kr ^ cl) << 2));
      float v[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (e.bias) v[r] = v[r] + rb[r];
        if constexpr (CT == kAnyC) {
          if (e.beta != 0.f) v[r] = __builtin_fmaf(e.beta, cur[u][r], v[r]);
        } else if constexpr (CT != -1) {
          v[r] = __builtin_fmaf(e.beta, cur[u][r], v[r]);
        }
      }
      const bool valid = !EDGE || (j < n && rowv);  // edge tiles: these 4 outputs are inside D, or none is
      if (amax) {
        if (valid) {
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = amax_fold(mx, v[r]);
        }
        asm volatile("" : "+v"(mx));  // folded here: sunk to the end, it keeps every value alive (spills)
      }
      if constexpr (EDGE) {
        if (!valid) continue;
      }
      if constexpr (DT == kAnyD) {
        store4_any(e.d_dtype, e.d, (size_t)j * e.ldd + i, v, qs);  // D 4-element aligned (class precondition)
      } else {
        uint8_t *dp = (uint8_t *)e.d + ((size_t)j * e.ldd + i) * elem_bytes(DT);
        if constexpr (DT == E5MA_FP32) {
          __builtin_nontemporal_store(v4f{v[0], v[1], v[2], v[3]}, (v4f *)dp);
        } else if constexpr (is_fp8(DT)) {
          __builtin_nontemporal_store(f32x4_to_fp8<DT>(v[0] * qs, v[1] * qs, v[2] * qs, v[3] * qs), (uint32_t *)dp);
        } else {
          __builtin_nontemporal_store(v2u{encode_t<DT>(v[0], 1.f) | encode_t<DT>(v[1], 1.f) << 16,
                                          encode_t<DT>(v[2], 1.f) | encode_t<DT>(v[3], 1.f) << 16},
                                      (v2u *)dp);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (CT != -1) load_group(0, ca);
  // pass h (a compile-time constant: it selects accumulator blocks, which must not be indexed at run time)
  auto pass = [&](auto hc) {
    constexpr int h = decltype(hc)::value;
    __syncthreads();  // the ring is free: the K loop's fragments, or the previous half, have been read
    {
#pragma unroll
      for (int yy = 0; yy < 2; ++yy) {
        const int y = 2 * h + yy;
        const int jt = 128 * wn + 32 * y + (lane & 31);  // tile column
        float sbj = sb1;
        if (e.sb_vec) sbj = e.sb[EDGE ? min(j0 + jt, n - 1) : j0 + jt];  // past n: never stored
        // pass column 64 wn + 32 yy + lane % 32, in buffer 4 wn + 2 yy + (lane & 16 ? 1 : 0): a select between
        // two pointers, not a lane-indexed switch
        const int b0 = 4 * wn + 2 * yy;
        float *colp = ((lane & 16) ? stage_at(b0 + 1) : stage_at(b0)) + lc * 256;
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_barrier(0);
            const int chunk = 32 * wm + 8 * x + 2 * g + hi;  // rows 4 chunk .. + 3
            float v[4];
            if (vs) {
              float as[4];
              if (e.sa_vec) {
                // rows past m (edge tiles; m % 4 == 0) read the last in-range group: never stored
                const float4 a4 = *(const float4 *)(e.sa + (EDGE ? min(i0 + 4 * chunk, m - 4) : i0 + 4 * chunk));
                as[0] = e.alpha * a4.x; as[1] = e.alpha * a4.y; as[2] = e.alpha * a4.z; as[3] = e.alpha * a4.w;
              } else {
                as[0] = as[1] = as[2] = as[3] = sa1;
              }
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * (as[q] * sbj);
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * s;
            }
            *(float4 *)(colp + ((chunk ^ lc) << 2)) = make_float4(v[0], v[1], v[2], v[3]);
          }
      }
    }
    __syncthreads();
    write_group(h, 0, ca, cb);
    write_group(h, 1, cb, ca);
    write_group(h, 2, ca, cb);
    write_group(h, 3, cb, ca);
  };
  pass(std::integral_constant<int, 0>{});
  pass(std::integral_constant<int, 1>{});
  return mx;
}

// Tiles at the m / n edges (or unaligned D): half a tile at a time -- the 128 columns of the waves with
// wn == h, 256 x 128 FP32 = the whole ring, column group c (16 columns) in ring buffer c -- is staged in
// LDS, then the block writes it out with bounds checks (general_half, dtypes at run time).
__device__ __forceinline__ float edge_epilogue(const TileArgs &t, const Epilogue &e, v16f (&acc)[4][4], int i0, int j0,
                                               int wm, int wn, int lane, int tid, int vec) {
  float mx = 0.f;
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
    mx = general_half<kAnyD, kAnyC>(e, st, t, i, j0 + 128 * h, rs, rb, vec, tid, mx);
  }
  return mx;
}


// The epilogue of a 256 x 128 half tile (waves of 128 x 64: accumulator blocks y < 2): the whole tile in
// FP32 is the ring, column c at buffer c / 16 as in edge_epilogue, written out once with bounds checks.
__device__ __forceinline__ float half_tile_epilogue(const TileArgs &t, const Epilogue &e, v16f (&acc)[4][4], int i0,
                                                    int j0, int wm, int wn, int lane, int tid, int vec) {
  float mx = 0.f;
  const EpiState st = epi_begin(e);
  const int i = i0 + 4 * (tid & 63);  // this thread's 4 rows in the write-out
  float rs[4], rb[4];                 // alpha * sa[i], bias[i] of those rows
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int iq = min(i + q, t.m - 1);
    rs[q] = e.alpha * (e.sa_vec ? e.sa[iq] : scale_or_one(e.sa));
    rb[q] = e.bias ? load_any(e.bias_dtype, e.bias, (size_t)iq, 1.f) : 0.f;
  }
  __syncthreads();  // the K loop no longer reads the ring
#pragma unroll
  for (int y = 0; y < 2; ++y) {
    // column 64 wn + 32 y + lane % 32: buffer 4 wn + 2 y + (lane & 16 ? 1 : 0), column lane % 16 in it
    float *grp = (lane & 16) ? stage_at(4 * wn + 2 * y + 1) : stage_at(4 * wn + 2 * y);
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
  __syncthreads();
  return general_half<kAnyD, kAnyC>(e, st, t, i, j0, rs, rb, vec, tid, mx);
}

// FP8 output (E4M3 / E5M2), no bias, beta = 0, 16-byte aligned D columns (ldd % 16 == 0), m % 16 == 0:
// the tile is staged once, as FP8 codes (64 KiB: 256 columns of 256 bytes, 64 columns per ring buffer),
// in place of staged_general's two passes of FP32 values.
// Phase W: v = acc * ((alpha * sa[i]) * sb[j]); amax; the codes of v * scale, one word per register
// group g (rows 8 g + 4 (l / 32) .. + 3 of lane l's column).  Two v_permlane32_swap, (g0, g2) and (g1, g3),
// give lane l rows 0..15 and lane l + 32 rows 16..31 of its 32-row block: 16 bytes, written to the
// column's 256 bytes at chunk k ^ (column % 16), so that the 16 lanes a ds_write_b128 serves per cycle
// meet 16 distinct bank groups.
// Phase R: step q writes tile columns 16 q .. 16 q + 15, thread t column 16 q + t / 16, rows
// 16 (t % 16) .. + 15 (16 threads per 256-byte column); the ring is read 8 steps at a time before the
// stores.  EDGE: stores and amax limited to D (m % 16 == 0, so a 16-row chunk lies inside or outside).
// A / B in the bench on one box: TE dgrad (N, N) 4096 x 8192 x 14336 to E5M2 with scale, amax and row-wise
// scale_inv 0.347 -> 0.325 ms; the other lines unchanged (TE wgrad -1.6 %: the class's copy now spills 3
// registers in place of 5).
template <int DT, bool EDGE>
__device__ __forceinline__ float staged8(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int m, int n, int wm,
                                         int wn, int lane, int tid, float sa1, float sb1) {
  const float s = sa1 * sb1, qs = scale_or_one(e.d_scale);
  const bool amax = e.amax != nullptr, sav_on = e.sa_vec;
  const int lc = lane & 31, hi = lane >> 5;
  float mx = 0.f;
  // this lane's row-group scales alpha * sa[i] (16 groups of 4 rows), loaded before the ring is free
  float4 sav[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int r4 = i0 + 128 * wm + 32 * x + 8 * g + 4 * hi;  // rows r4 .. r4 + 3
      if (sav_on) {
        // rows past m (edge tiles) read the last in-range group: never stored
        const float4 a4 = *(const float4 *)(e.sa + (EDGE ? min(r4, m - 4) : r4));
        sav[x][g] = make_float4(e.alpha * a4.x, e.alpha * a4.y, e.alpha * a4.z, e.alpha * a4.w);
      } else {
        sav[x][g] = make_float4(sa1, sa1, sa1, sa1);
      }
    }
  __syncthreads();  // every wave has read its last fragments from the ring
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int jt = 128 * wn + 32 * y + lc;  // tile column
    const bool colv = !EDGE || j0 + jt < n;
    float sbj = sb1;
    if (e.sb_vec) sbj = e.sb[EDGE ? min(j0 + jt, n - 1) : j0 + jt];  // past n: never stored
    uint8_t *col = (uint8_t *)stage_at(2 * wn + (y >> 1)) + (32 * (y & 1) + lc) * 256;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      __builtin_amdgcn_sched_barrier(0);
      uint32_t w[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
        if (e.sa_vec || e.sb_vec) {
          const float as[4] = {sav[x][g].x, sav[x][g].y, sav[x][g].z, sav[x][g].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * (as[q] * sbj);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc_read(acc[x][y][4 * g + q]) * s;
        }
        if (amax) {
          if (!EDGE || (colv && i0 + 128 * wm + 32 * x + 8 * g + 4 * hi < m)) {
#pragma unroll
            for (int q = 0; q < 4; ++q) mx = amax_fold(mx, v[q]);
          }
        }
        w[g] = f32x4_to_fp8<DT>(v[0] * qs, v[1] * qs, v[2] * qs, v[3] * qs);
      }
      const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
      const int k = 8 * wm + 2 * x + hi;  // the lane's 16-row chunk of the column after the swaps
      *(uint4 *)(col + ((k ^ (lc & 15)) << 4)) = make_uint4(s0[0], s0[1], s1[0], s1[1]);
    }
  }
  if (amax) asm volatile("" : "+v"(mx));
  __syncthreads();
  // phase R
  const int cq = tid >> 4, k = tid & 15;
  const bool rowv = !EDGE || i0 + 16 * k < m;
  uint8_t *gp = (uint8_t *)e.d + (size_t)(j0 + cq) * e.ldd + i0 + 16 * k;
  const size_t gstep = (size_t)16 * e.ldd;  // 16 columns
  constexpr int kBatch = EDGE ? 1 : 8;
#pragma unroll
  for (int q0 = 0; q0 < 16; q0 += kBatch) {
    uint4 d[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int q = q0 + u, cl = 16 * (q & 3) + cq;  // column within ring buffer q / 4
      d[u] = *(const uint4 *)((const uint8_t *)stage_at(q >> 2) + cl * 256 + ((k ^ cq) << 4));
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int q = q0 + u;
      if (!EDGE || (rowv && j0 + 16 * q + cq < n)) *(uint4 *)(gp + q * gstep) = d[u];
    }
  }
  return mx;
}

// Epilogue classes, one kernel instance each (kernels holding every epilogue spill registers, and the
// spills cost the headline GEMM 4.6%): kEpiFast16 -- no bias, beta = 0, no amax, a BF16 D with 16-byte
// aligned columns, m % 8 == 0 (staged16); kEpiFull -- 4-element aligned D and C, m % 4 == 0
// (staged_general; FP16 D and amax too; an FP8 D with 16-byte aligned columns, m % 16 == 0 and no bias
// or C: staged8); kEpiAny -- unaligned D or C, or m % 4 != 0,
// every tile through the half-tile write-out with bounds checks and run-time dtypes (edge_epilogue).  The
// staged write-outs take edge tiles themselves (the bounds-checked path had cost an edge tile ~30 us,
// and a round waits for its slowest tile: 8000^2 x 8192 took 555 us against 399 us for 8192^2).
constexpr int kEpiFast16 = 0, kEpiFull = 1, kEpiAny = 2;

// the class a launch takes (host side)
inline int epilogue_class(int m, int n, const Epilogue &e, int simple, int vec) {
  (void)n;  // the staged write-outs take edge tiles too
  if (simple && e.d_dtype == E5MA_BF16 && e.amax == nullptr && (uintptr_t)e.d % 16 == 0 && e.ldd % 8 == 0 &&
      m % 8 == 0)
    return kEpiFast16;
  const bool c_ok = e.beta == 0.f || ((uintptr_t)e.c % (4 * elem_bytes(e.c_dtype)) == 0 && e.ldc % 4 == 0);
  return vec && c_ok && m % 4 == 0 ? kEpiFull : kEpiAny;  // m % 4: a thread's 4 rows never straddle m
}

// staged_general for D / C dtypes chosen at run time (the common pairings have their own instances)
template <bool EDGE>
__device__ __forceinline__ float staged_full(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int m, int n, int wm,
                                             int wn, int lane, int tid, float sa1, float sb1) {
  const int dt = e.d_dtype, c = e.beta != 0.f ? e.c_dtype : -1;
  // FP8 D without bias or C, 16-byte aligned columns (launch-uniform): staged as codes
  if (c == -1 && e.bias == nullptr && (uintptr_t)e.d % 16 == 0 && e.ldd % 16 == 0 && m % 16 == 0) {
    if (dt == E5MA_E5M2) return staged8<E5MA_E5M2, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
    if (dt == E5MA_E4M3) return staged8<E5MA_E4M3, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
  }
  if (dt == E5MA_FP32 && c == E5MA_FP32)
    return staged_general<E5MA_FP32, E5MA_FP32, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
  if (c == -1) {
    if (dt == E5MA_FP32) return staged_general<E5MA_FP32, -1, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
    if (dt == E5MA_BF16) return staged_general<E5MA_BF16, -1, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
    if (dt == E5MA_E5M2) return staged_general<E5MA_E5M2, -1, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
    if (dt == E5MA_E4M3) return staged_general<E5MA_E4M3, -1, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
  }
  return staged_general<kAnyD, kAnyC, EDGE>(e, acc, i0, j0, m, n, wm, wn, lane, tid, sa1, sb1);
}

// Persistent launches (block b takes tiles b, b + gridDim.x, ...): a block with no tile in the launch's last
// round (a partly filled last round) starts about half a tile late, waiting wait_cycles on the shader clock.
// The write-outs of the two groups of blocks then come at different times instead of all at once (TE wgrad
// 14336 x 4096 x 8192, 896 tiles: 417.7 -> 409.4 us), and the late blocks still finish first.
__device__ __forceinline__ void late_start(const TileArgs &t, unsigned long long wait_cycles) {
  const int mine = (t.count - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int most = (t.count + (int)gridDim.x - 1) / (int)gridDim.x;
  if (mine < most) {
    const unsigned long long s0 = __builtin_amdgcn_s_memtime();
    while (__builtin_amdgcn_s_memtime() - s0 < wait_cycles) __builtin_amdgcn_s_sleep(32);
  }
}

// The epilogue of a block tile (acc: this wave's accumulators; i0, j0: the tile's origin; sa1 = alpha * sa
// and sb1 = sb, the per-tensor scales read before the K loop) for D of any dtype (e.d_dtype), in class
// EPI.  Returns the thread's max |value| for amax.
template <int EPI>
__device__ __forceinline__ float tile_epilogue(const TileArgs &t, const Epilogue &e, v16f (&acc)[4][4], int i0, int j0,
                                               int wm, int wn, int lane, int tid, int simple, int vec, float sa1,
                                               float sb1) {
  // (a scheduling barrier keeps the compiler from hoisting epilogue work into the K loop's tail)
  __builtin_amdgcn_sched_barrier(0);
  const bool full = i0 + kBM <= t.m && j0 + kBN <= t.n;  // block-uniform
  if constexpr (EPI == kEpiFast16) {
    const bool vs = e.sa_vec || e.sb_vec;  // launch-uniform
    if (full) {
      if (vs) staged16<false, true>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
      else staged16<false, false>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
    } else {
      if (vs) staged16<true, true>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
      else staged16<true, false>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
    }
    return 0.f;  // no amax in this class
  } else if constexpr (EPI == kEpiFull) {
    if (full) return staged_full<false>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
    return staged_full<true>(e, acc, i0, j0, t.m, t.n, wm, wn, lane, tid, sa1, sb1);
  } else {
    (void)simple;
    return edge_epilogue(t, e, acc, i0, j0, wm, wn, lane, tid, vec);
  }
}

}  // namespace tile
}  // namespace
}  // namespace e5ma
