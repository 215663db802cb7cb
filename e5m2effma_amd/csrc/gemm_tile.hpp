// gemm_tile.hpp -- what the matrix-core tile kernels (gemm_f8_kernel.hpp, gemm_h_kernel.hpp) share:
// the 256 x 256 block tile of 4 waves (128 x 128 accumulators each, 4 x 4 blocks of 32 x 32), the
// 128 KiB LDS ring of 8 buffers and its direct-to-LDS loads, the XCD-aware tile order, and the epilogue.
#pragma once
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
};

// Output tile and K split of block b.  XCD-aware when the block count is a multiple of 8 (blocks are
// dispatched to the 8 XCDs round-robin): an XCD runs consecutive indices x, so with K splits each XCD
// works on one split (one K slice of the operands in its L2); then tiles are grouped kGroupM m-tiles
// at a time.
__device__ __forceinline__ void tile_of(int b, const TileArgs &t, int &tm, int &tn, int &split) {
  const int tiles = t.tiles_m * t.tiles_n, total = tiles * t.splits;
  int x = b;
  if ((total & 7) == 0) x = (b & 7) * (total >> 3) + (b >> 3);
  split = x / tiles;
  x -= split * tiles;
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

// Writes out one staged half tile (256 rows x 128 columns starting at column jh) in the reference's
// epilogue order (include/e5m2effma.h: v = acc * (alpha * sa[i]) * sb[j]; v += bias[i];
// v = fma(beta, C * csinv, v); amax; convert).  Wave w takes columns w, w + 4, ..., thread t rows
// i .. i + 3 (i = i0 + 4 (t % 64)); eight columns per step, with their C values loaded (one vector load
// per column when C is aligned) before any is computed or stored, so 32 values per thread are in
// flight (C may alias D: each element is read before it is written, by the same thread).  CT: the
// dtype of C, or -1 when beta = 0.
template <int DT, int CT>
__device__ __forceinline__ float general_half(const Epilogue &e, const EpiState &st, const TileArgs &t, int i, int jh,
                                              const float (&rs)[4], const float (&rb)[4], int vec, int tid,
                                              float mx) {
  constexpr int kCols = 8;  // columns per step
  const int w = tid >> 6, il = 4 * (tid & 63);
  const bool rows4 = i + 3 < t.m;
  bool cvec = false;
  if constexpr (CT >= 0)
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
      if constexpr (CT >= 0) {
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

// Four BF16 codes (v[0] in the lowest half) by the hardware's pair conversion v_cvt_pk_bf16_f32: checked
// here against the integer round-to-nearest-even encoder over all 2^32 FP32 inputs, identical except for
// NaNs, which it keeps NaN but with their sign and payload.  Every NaN must become 0x7FC0
// (include/e5m2effma.h, reference rne_hi), so lanes holding one take a rarely executed fix-up: the
// common path is 4 compares and 2 conversions per 4 values (the integer encoder costs about 6 per value).
__device__ __forceinline__ uint2 bf16_quad(const float (&v)[4]) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  uint32_t lo = __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)v[0], (__bf16)v[1]});
  uint32_t hi = __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)v[2], (__bf16)v[3]});
  // the flags are taken before the branch, so the values are dead across it (else they are spilled)
  const bool n0 = v[0] != v[0], n1 = v[1] != v[1], n2 = v[2] != v[2], n3 = v[3] != v[3];
  if (n0 || n1 || n2 || n3) {
    if (n0) lo = (lo & 0xFFFF0000u) | 0x7FC0u;
    if (n1) lo = (lo & 0x0000FFFFu) | 0x7FC00000u;
    if (n2) hi = (hi & 0xFFFF0000u) | 0x7FC0u;
    if (n3) hi = (hi & 0x0000FFFFu) | 0x7FC00000u;
  }
  return make_uint2(lo, hi);
}

// The direct epilogue of a full tile with no bias and beta = 0: scale, convert and store straight from
// the accumulators, column by column (y outer): the 16 stores into one column's cache lines follow each
// other, so the L2 writes the lines back whole (x / g outer measured 3x the write traffic).  AMAX: fold
// |value| for amax (compiled out otherwise: the epilogue is VALU-bound with one wave per SIMD).
template <int DT, bool AMAX>
__device__ __forceinline__ float direct_epilogue(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int wm, int wn,
                                                 int lane) {
  float mx = 0.f;
  const EpiState st = epi_begin(e);
  const int ib0 = i0 + 128 * wm + 4 * (lane >> 5);
  const float sa1 = e.alpha * scale_or_one(e.sa), sb1 = scale_or_one(e.sb);
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
          if constexpr (AMAX) mx = amax_fold(mx, v[q]);
        }
        uint8_t *dp = colp + (32 * x + 8 * g) * elem_bytes(DT);
        if constexpr (DT == E5MA_FP32) {
          *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
        } else if constexpr (is_fp8(DT)) {
          *(uint32_t *)dp = encode_t<DT>(v[0], st.qscale) | encode_t<DT>(v[1], st.qscale) << 8 |
                            encode_t<DT>(v[2], st.qscale) << 16 | encode_t<DT>(v[3], st.qscale) << 24;
        } else if constexpr (DT == E5MA_BF16) {
          *(uint2 *)dp = bf16_quad(v);
        } else {
          *(uint2 *)dp = make_uint2(encode_t<DT>(v[0], 1.f) | encode_t<DT>(v[1], 1.f) << 16,
                                    encode_t<DT>(v[2], 1.f) | encode_t<DT>(v[3], 1.f) << 16);
        }
      }
  }
  return mx;
}

// The direct epilogue of a full tile with a bias and / or beta * C (C of dtype CT, -1 when beta = 0, with
// 4-element aligned columns): the direct epilogue's layout and column order, with C read in that same
// layout, 16 bytes (FP32) per lane and (x, g).  Units u = 4 y + x (4 loads each, g = 0..3) stream
// through a ring of kSlots units, refilled as each unit is consumed: 24 loads per lane in flight
// (96 VGPRs), where staging through LDS, 8 columns per thread per step, kept a third of that in flight.
// The bias of the tile's 256 rows goes to LDS once (FP32).  Same operation order as general_half:
// v = acc * ((alpha * sa[i]) * sb[j]); v + bias[i]; fma(beta, C, v).  C may alias D: each element is
// loaded before the same thread stores it.  All threads of the block must call it (two barriers).
template <int DT, int CT>
__device__ __forceinline__ float direct_general(const Epilogue &e, v16f (&acc)[4][4], int i0, int j0, int wm, int wn,
                                                int lane, int tid) {
  constexpr int kSlots = 6;
  float mx = 0.f;
  const EpiState st = epi_begin(e);
  const int ib0 = i0 + 128 * wm + 4 * (lane >> 5);
  const float sa1 = e.alpha * scale_or_one(e.sa), sb1 = scale_or_one(e.sb);
  float *bias_lds = stage_at(0);
  __syncthreads();  // the ring is no longer read
  bias_lds[tid] = e.bias ? load_any(e.bias_dtype, e.bias, (size_t)(i0 + tid), 1.f) : 0.f;
  __syncthreads();
  float cv[kSlots][4][4];
  const auto load_unit = [&](int u, float (&c)[4][4]) {
    const int y = u >> 2, x = u & 3;
    const size_t at = (size_t)(j0 + 128 * wn + 32 * y + (lane & 31)) * e.ldc + ib0 + 32 * x;
#pragma unroll
    for (int g = 0; g < 4; ++g) load4_t<CT>(e.c, at + 8 * g, st.csinv, c[g]);
  };
  if constexpr (CT >= 0) {
#pragma unroll
    for (int u = 0; u < kSlots; ++u) load_unit(u, cv[u]);
  }
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int y = u >> 2, x = u & 3;
    const int j = j0 + 128 * wn + 32 * y + (lane & 31);
    const float sbj = e.sb_vec ? e.sb[j] : sb1;
    uint8_t *colp = (uint8_t *)e.d + ((size_t)j * e.ldd + ib0 + 32 * x) * elem_bytes(DT);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      const int il = 128 * wm + 32 * x + 8 * g + 4 * (lane >> 5);
      const float4 b4 = *(const float4 *)(bias_lds + il);
      const float rb[4] = {b4.x, b4.y, b4.z, b4.w};
      float as[4];
      if (e.sa_vec) {
        const float4 v = *(const float4 *)(e.sa + i0 + il);
        as[0] = e.alpha * v.x; as[1] = e.alpha * v.y; as[2] = e.alpha * v.z; as[3] = e.alpha * v.w;
      } else {
        as[0] = as[1] = as[2] = as[3] = sa1;
      }
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float sc = (e.sa_vec || e.sb_vec) ? as[q] * sbj : st.s;
        v[q] = acc_read(acc[x][y][4 * g + q]) * sc;
        if (e.bias) v[q] = v[q] + rb[q];
        if constexpr (CT >= 0) v[q] = __builtin_fmaf(e.beta, cv[u % kSlots][g][q], v[q]);
        mx = amax_fold(mx, v[q]);
      }
      uint8_t *dp = colp + 8 * g * elem_bytes(DT);
      if constexpr (DT == E5MA_FP32) {
        *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
      } else if constexpr (is_fp8(DT)) {
        *(uint32_t *)dp = encode_t<DT>(v[0], st.qscale) | encode_t<DT>(v[1], st.qscale) << 8 |
                          encode_t<DT>(v[2], st.qscale) << 16 | encode_t<DT>(v[3], st.qscale) << 24;
      } else if constexpr (DT == E5MA_BF16) {
        *(uint2 *)dp = bf16_quad(v);
      } else {
        *(uint2 *)dp = make_uint2(encode_t<DT>(v[0], 1.f) | encode_t<DT>(v[1], 1.f) << 16,
                                  encode_t<DT>(v[2], 1.f) | encode_t<DT>(v[3], 1.f) << 16);
      }
    }
    // unit u's slot is free: refill it with unit u + kSlots
    if constexpr (CT >= 0) {
      __builtin_amdgcn_sched_barrier(0);
      if (u + kSlots < 16) load_unit(u + kSlots, cv[u % kSlots]);
    }
  }
  return mx;
}

// The epilogue of a block tile (acc: this wave's accumulators; i0, j0: the tile's origin).  Returns the
// thread's max |value| for amax.
template <int DT>
__device__ __forceinline__ float tile_epilogue(const TileArgs &t, const Epilogue &e, v16f (&acc)[4][4], int i0, int j0,
                                               int wm, int wn, int lane, int tid, int simple, int vec) {
  // ---- epilogue.  Lane l, register r of block (x, y): output
  //   i = i0 + 128*wm + 32*x + 8*(r/4) + 4*(l/32) + r%4,  j = j0 + 128*wn + 32*y + l%32
  // (scheduling barriers keep the compiler from hoisting epilogue work into the K loop's tail and from
  // copying all accumulators to VGPRs at once, both of which spill)
  __builtin_amdgcn_sched_barrier(0);
  float mx = 0.f;
  if (simple && i0 + kBM <= t.m && j0 + kBN <= t.n) {
    // no bias, beta = 0, a full tile, D aligned for 4-element stores
    mx = e.amax ? direct_epilogue<DT, true>(e, acc, i0, j0, wm, wn, lane)
                : direct_epilogue<DT, false>(e, acc, i0, j0, wm, wn, lane);
  } else if (vec && i0 + kBM <= t.m && j0 + kBN <= t.n &&
             (e.beta == 0.f ||
              (e.c_dtype == E5MA_FP32 && (uintptr_t)e.c % 16 == 0 && e.ldc % 4 == 0))) {
    // a full tile with a bias and / or beta * FP32 C (TE's wgrad into main_grad), D and C aligned
    mx = e.beta != 0.f ? direct_general<DT, E5MA_FP32>(e, acc, i0, j0, wm, wn, lane, tid)
                       : direct_general<DT, -1>(e, acc, i0, j0, wm, wn, lane, tid);
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
  return mx;
}

}  // namespace tile
}  // namespace
}  // namespace e5ma
