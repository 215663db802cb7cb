// e5ma_device.hpp -- device-side numerics shared by the gfx950 kernels: FP8 / BF16 / FP16 codecs,
// typed element access, the wave64 amax reduction and the GEMM / GEMV epilogue.
//
// Every conversion is exact integer arithmetic written from the format definitions (OCP FP8 E5M2 /
// E4M3, bfloat16, IEEE binary16), so results are bit-identical to the reference's device numerics
// (reference src/e5m2effma.cuh:43-124) independent of the hardware's conversion modes.  The hot
// kernels may use the hardware packed converts instead where a test pins them to these.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e5m2effma.h"

namespace e5ma {

__host__ __device__ constexpr bool is_fp8(int t) { return t == E5MA_E5M2 || t == E5MA_E4M3; }
__host__ __device__ constexpr int elem_bytes(int t) { return is_fp8(t) ? 1 : t == E5MA_FP32 ? 4 : 2; }

namespace dev {

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// ---- decoders ---------------------------------------------------------------------------------
// E5M2 is the upper byte of an IEEE binary16 (reference src/e5m2effma.cuh:69-72): exact; the Inf
// codes decode to +-Inf, every NaN code to the NaN 0x7FFFFFFF (what the reference's hardware
// half-to-float convert produces).
__device__ __forceinline__ float e5m2_value(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24, e = (b >> 2) & 31u, f = b & 3u;
  if (e == 31u) return f ? u2f(0x7FFFFFFFu) : u2f(s | 0x7F800000u);
  if (e == 0u) return u2f(s | f2u((float)f * 0x1p-16f));
  return u2f(s | ((e + 112u) << 23) | (f << 21));
}
// E4M3 ("fn": no Inf; S.1111.111 is NaN and decodes to 0x7FFFFFFF; reference src/e5m2effma.cuh:54-58).
__device__ __forceinline__ float e4m3_value(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24, e = (b >> 3) & 15u, f = b & 7u;
  if ((b & 0x7Fu) == 0x7Fu) return u2f(0x7FFFFFFFu);
  if (e == 0u) return u2f(s | f2u((float)f * 0x1p-9f));
  return u2f(s | ((e + 120u) << 23) | (f << 20));
}
__device__ __forceinline__ float bf16_value(uint32_t h) { return u2f(h << 16); }
__device__ __forceinline__ float f16_value(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---- encoders ---------------------------------------------------------------------------------
// FP32 -> BF16 bits, round to nearest even; every NaN -> 0x7FC0 (reference src/e5m2effma.cuh:80-88).
__device__ __forceinline__ uint32_t f32_to_bf16(float x) {
  const uint32_t u = f2u(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
// FP32 -> IEEE binary16 bits, round to nearest even (the hardware convert in the default mode).  The
// empty asm keeps the compiler from folding a preceding multiply into a mixed-precision multiply-add
// with a +0 addend, which would turn a -0 product into +0.
__device__ __forceinline__ uint32_t f32_to_f16(float x) {
  asm volatile("" : "+v"(x));
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}
// FP32 -> FP8 codes (E5M2: v_cvt_pk_bf8_f32, E4M3: v_cvt_pk_fp8_f32): round to nearest even, |x| >= the
// largest finite value (Inf included) saturates to it, every NaN -> 0x7F (sign dropped) -- the semantics of
// cvt.rn.satfinite used by the reference (src/e5m2effma.cuh:90-124).  The instructions do not saturate, so
// the input is first clamped to [-max, max] (v_med3_f32), and NaN is selected apart.  Equal, for every one of
// the 2^32 FP32 inputs, to the integer formulation rounding the significand at bit 23 - mantissa bits (with a
// subnormal grid of 2^(1 - bias - mantissa bits)), which this library used before: compared exhaustively on
// gfx950, both encoders and both words of the pair instruction.
template <int T> constexpr float kFp8Max = T == E5MA_E5M2 ? 57344.f : 448.f;
// codes of a and b into word HI of old (bytes 2 HI, 2 HI + 1), the other word kept
template <int T, bool HI> __device__ __forceinline__ uint32_t fp8_pair_into(float a, float b, uint32_t old) {
  const float ca = __builtin_amdgcn_fmed3f(a, -kFp8Max<T>, kFp8Max<T>);
  const float cb = __builtin_amdgcn_fmed3f(b, -kFp8Max<T>, kFp8Max<T>);
  if constexpr (T == E5MA_E5M2) return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(ca, cb, (int)old, HI);
  else return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, (int)old, HI);
}
// four codes, v0 in byte 0 .. v3 in byte 3
template <int T> __device__ __forceinline__ uint32_t f32x4_to_fp8(float v0, float v1, float v2, float v3) {
  uint32_t r = fp8_pair_into<T, true>(v2, v3, fp8_pair_into<T, false>(v0, v1, 0u));
  if (v0 != v0) r = (r & 0xFFFFFF00u) | 0x0000007Fu;
  if (v1 != v1) r = (r & 0xFFFF00FFu) | 0x00007F00u;
  if (v2 != v2) r = (r & 0xFF00FFFFu) | 0x007F0000u;
  if (v3 != v3) r = (r & 0x00FFFFFFu) | 0x7F000000u;
  return r;
}
template <int T> __device__ __forceinline__ uint32_t f32_to_fp8_code(float x) {
  return x != x ? 0x7Fu : fp8_pair_into<T, false>(x, x, 0u) & 0xFFu;
}
__device__ __forceinline__ uint32_t f32_to_e5m2(float x) { return f32_to_fp8_code<E5MA_E5M2>(x); }
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) { return f32_to_fp8_code<E5MA_E4M3>(x); }
template <int T> __device__ __forceinline__ uint32_t f32_to_fp8t(float x) {
  return T == E5MA_E5M2 ? f32_to_e5m2(x) : f32_to_e4m3(x);
}

// ---- typed element access (reference src/e5m2effma.cuh:131-153) ------------------------------
__device__ __forceinline__ float scale_or_one(const float *p) { return p ? *p : 1.0f; }

template <int T> __device__ __forceinline__ float load_t(const void *p, size_t i, float sinv) {
  if constexpr (T == E5MA_E5M2) return e5m2_value(((const uint8_t *)p)[i]) * sinv;
  else if constexpr (T == E5MA_E4M3) return e4m3_value(((const uint8_t *)p)[i]) * sinv;
  else if constexpr (T == E5MA_BF16) return bf16_value(((const uint16_t *)p)[i]);
  else if constexpr (T == E5MA_FP16) return f16_value(((const uint16_t *)p)[i]);
  else return ((const float *)p)[i];
}
__device__ __forceinline__ float load_any(int t, const void *p, size_t i, float sinv) {
  switch (t) {
    case E5MA_E5M2: return load_t<E5MA_E5M2>(p, i, sinv);
    case E5MA_E4M3: return load_t<E5MA_E4M3>(p, i, sinv);
    case E5MA_BF16: return load_t<E5MA_BF16>(p, i, sinv);
    case E5MA_FP16: return load_t<E5MA_FP16>(p, i, sinv);
    default: return load_t<E5MA_FP32>(p, i, sinv);
  }
}
// element code of v in dtype T (FP8: RNE satfinite of v * qscale)
template <int T> __device__ __forceinline__ uint32_t encode_t(float v, float qscale) {
  if constexpr (T == E5MA_E5M2) return f32_to_e5m2(v * qscale);
  else if constexpr (T == E5MA_E4M3) return f32_to_e4m3(v * qscale);
  else if constexpr (T == E5MA_BF16) return f32_to_bf16(v);
  else if constexpr (T == E5MA_FP16) return f32_to_f16(v);
  else return f2u(v);
}
template <int T> __device__ __forceinline__ void store_t(void *p, size_t i, float v, float qscale) {
  if constexpr (is_fp8(T)) ((uint8_t *)p)[i] = (uint8_t)encode_t<T>(v, qscale);
  else if constexpr (T == E5MA_FP32) ((float *)p)[i] = v;
  else ((uint16_t *)p)[i] = (uint16_t)encode_t<T>(v, qscale);
}
__device__ __forceinline__ void store_any(int t, void *p, size_t i, float v, float qscale) {
  switch (t) {
    case E5MA_E5M2: store_t<E5MA_E5M2>(p, i, v, qscale); break;
    case E5MA_E4M3: store_t<E5MA_E4M3>(p, i, v, qscale); break;
    case E5MA_BF16: store_t<E5MA_BF16>(p, i, v, qscale); break;
    case E5MA_FP16: store_t<E5MA_FP16>(p, i, v, qscale); break;
    default: store_t<E5MA_FP32>(p, i, v, qscale); break;
  }
}
// Four consecutive elements i .. i + 3 of dtype T (4-element aligned) in one vector store
template <int T> __device__ __forceinline__ void store4_t(void *p, size_t i, const float (&v)[4], float qscale) {
  uint8_t *dp = (uint8_t *)p + i * elem_bytes(T);
  if constexpr (T == E5MA_FP32) {
    *(float4 *)dp = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (is_fp8(T)) {
    *(uint32_t *)dp = f32x4_to_fp8<T>(v[0] * qscale, v[1] * qscale, v[2] * qscale, v[3] * qscale);
  } else {
    *(uint2 *)dp = make_uint2(encode_t<T>(v[0], qscale) | encode_t<T>(v[1], qscale) << 16,
                              encode_t<T>(v[2], qscale) | encode_t<T>(v[3], qscale) << 16);
  }
}
// the same with the dtype chosen at run time (one dispatch per four elements)
__device__ __forceinline__ void store4_any(int t, void *p, size_t i, const float (&v)[4], float qscale) {
  switch (t) {
    case E5MA_E5M2: store4_t<E5MA_E5M2>(p, i, v, qscale); break;
    case E5MA_E4M3: store4_t<E5MA_E4M3>(p, i, v, qscale); break;
    case E5MA_BF16: store4_t<E5MA_BF16>(p, i, v, qscale); break;
    case E5MA_FP16: store4_t<E5MA_FP16>(p, i, v, qscale); break;
    default: store4_t<E5MA_FP32>(p, i, v, qscale); break;
  }
}

// ---- amax ---------------------------------------------------------------------------------------
// Folds |v| into a running maximum, ignoring every NaN (quiet or signalling): the comparison is false
// for NaN.  fmaxf is not used here: in IEEE mode a signalling NaN input makes it return NaN, which
// would discard the maximum gathered so far.
__device__ __forceinline__ float amax_fold(float m, float v) {
  const float a = fabsf(v);
  return a > m ? a : m;
}
// max over the 64 lanes of a wave (fmaxf ignores NaN, as the reference's reduction does)
__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
  for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  return m;
}
// Block-wide max of each thread's m, then one atomicMax of the float bits into *amax, issued only
// for a positive maximum: non-negative floats order like their bit patterns, and the value already
// in *amax is max-reduced with it (reference src/e5m2effma.cuh:190-195).  All threads of the block
// must call it; red holds blockDim.x / 64 floats of LDS.
__device__ __forceinline__ void amax_commit_block(float *amax, float m, float *red) {
  m = wave_max(m);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = red[0];
    for (int i = 1; i < nw; ++i) b = fmaxf(b, red[i]);
    // With many blocks, most maxima are below the value already in *amax: skip their atomics.  The
    // read may be stale, which only costs an atomic; the atomicMax alone decides the result.
    if (b > 0.f && __float_as_int(b) > __atomic_load_n((const int *)amax, __ATOMIC_RELAXED))
      atomicMax((int *)amax, __float_as_int(b));
  }
}

// ---- GEMM / GEMV epilogue (include/e5m2effma.h:29-31; reference src/e5m2effma.cuh:198-241) -------
struct Epilogue {
  const float *sa, *sb;  // scale_inv of FP8 A / B (NULL = 1)
  int sa_vec, sb_vec;    // sa[i] per row of op(A) / sb[j] per column of op(B)
  float alpha, beta;
  const void *c;
  long long ldc;
  int c_dtype;
  const float *c_sinv;
  void *d;
  long long ldd;
  int d_dtype;
  const float *d_scale;
  float *amax;
  const void *bias;
  int bias_dtype;
};

struct EpiState {
  float s, qscale, csinv;
};

__device__ __forceinline__ EpiState epi_begin(const Epilogue &e) {
  EpiState st;
  st.s = (e.alpha * scale_or_one(e.sa)) * scale_or_one(e.sb);
  st.qscale = scale_or_one(e.d_scale);
  st.csinv = scale_or_one(e.c_sinv);
  return st;
}
// (alpha * sa[i]) * sb[j]
__device__ __forceinline__ float epi_scale(const Epilogue &e, const EpiState &st, int i, int j) {
  if (!e.sa_vec && !e.sb_vec) return st.s;
  const float a = e.sa_vec ? e.sa[i] : scale_or_one(e.sa);
  const float b = e.sb_vec ? e.sb[j] : scale_or_one(e.sb);
  return (e.alpha * a) * b;
}
// FP32 value of output (i, j) before conversion: v = acc * s; v += bias[i]; v = fma(beta, C * csinv, v).
// C may alias D: the caller reads C and writes D from the same thread.
__device__ __forceinline__ float epi_value(const Epilogue &e, const EpiState &st, int i, int j, float acc) {
  float v = acc * epi_scale(e, st, i, j);
  if (e.bias) v = v + load_any(e.bias_dtype, e.bias, (size_t)i, 1.f);
  if (e.beta != 0.f) v = __builtin_fmaf(e.beta, load_any(e.c_dtype, e.c, (size_t)j * e.ldc + i, st.csinv), v);
  return v;
}

}  // namespace dev
}  // namespace e5ma
