// vec.hpp -- 16-byte-vector element packs for the streaming kernels (cast, Adam): N consecutive
// elements of dtype T held as dwordx4 words, decoded to / encoded from FP32.
#pragma once
#include "e5ma_device.hpp"

namespace e5ma {
namespace dev {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// N elements of dtype T as N * bytes(T) / 16 dwordx4 words (N * bytes(T) must be a multiple of 8).
// NT: 16-byte accesses are non-temporal (data touched once).
template <int T, int N, bool NT = false> struct Pack {
  static constexpr int kBytes = N * elem_bytes(T);
  static constexpr int kWords = kBytes / 4;
  uint32_t w[kWords];

  __device__ __forceinline__ void load(const void *base, size_t i) {
    const uint8_t *p = (const uint8_t *)base + i * elem_bytes(T);
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int q = 0; q < kBytes / 16; ++q) {
        const u32x4 v = NT ? __builtin_nontemporal_load((const u32x4 *)p + q) : ((const u32x4 *)p)[q];
        w[4 * q] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int q = 0; q < kBytes / 8; ++q) {
        const uint2 v = ((const uint2 *)p)[q];
        w[2 * q] = v.x; w[2 * q + 1] = v.y;
      }
    }
  }
  __device__ __forceinline__ void store(void *base, size_t i) const {
    uint8_t *p = (uint8_t *)base + i * elem_bytes(T);
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int q = 0; q < kBytes / 16; ++q) {
        const u32x4 v{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
        if constexpr (NT) __builtin_nontemporal_store(v, (u32x4 *)p + q);
        else ((u32x4 *)p)[q] = v;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kBytes / 8; ++q) ((uint2 *)p)[q] = make_uint2(w[2 * q], w[2 * q + 1]);
    }
  }
  // element e as FP32 (FP8 times sinv; the others exact)
  __device__ __forceinline__ float get(int e, float sinv) const {
    if constexpr (is_fp8(T)) {
      const uint32_t b = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
      return (T == E5MA_E5M2 ? e5m2_value(b) : e4m3_value(b)) * sinv;
    } else if constexpr (T == E5MA_FP32) {
      return u2f(w[e]);
    } else {
      const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      return T == E5MA_BF16 ? bf16_value(h) : f16_value(h);
    }
  }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int q = 0; q < kWords; ++q) w[q] = 0;
  }
  // every element from v (FP8: four codes per conversion pair of instructions)
  __device__ __forceinline__ void set(const float (&v)[N], float qscale) {
    if constexpr (is_fp8(T) && N % 4 == 0) {
#pragma unroll
      for (int q = 0; q < N / 4; ++q)
        w[q] = f32x4_to_fp8<T>(v[4 * q] * qscale, v[4 * q + 1] * qscale, v[4 * q + 2] * qscale, v[4 * q + 3] * qscale);
    } else {
      clear();
#pragma unroll
      for (int e = 0; e < N; ++e) put(e, v[e], qscale);
    }
  }
  // set element e (freshly cleared pack) to the code of v
  __device__ __forceinline__ void put(int e, float v, float qscale) {
    const uint32_t c = encode_t<T>(v, qscale);
    if constexpr (is_fp8(T)) w[e >> 2] |= c << (8 * (e & 3));
    else if constexpr (T == E5MA_FP32) w[e] = c;
    else w[e >> 1] |= c << (16 * (e & 1));
  }
};

}  // namespace dev
}  // namespace e5ma
