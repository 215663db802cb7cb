// cast.hip -- e5ma_cast: dst = convert(src * sinv), amax = max |src * sinv| (reference
// src/e5m2effma.cu:53-63).  HBM-bound streaming kernel: 16 elements per thread per step through
// dwordx4 loads and stores when both buffers are 16-byte aligned, element by element otherwise
// (both paths convert each element identically).
#include "e5ma_host.hpp"
#include "vec.hpp"

namespace e5ma {
namespace {

using namespace dev;
constexpr int kThreads = 256;
constexpr int kVec = 16;
// Non-temporal accesses per side (measured on 8192^2 FP32 -> E5M2: ordinary loads and stores 61.5 us,
// non-temporal stores only 59.3 us, non-temporal loads only 83.0 us, both non-temporal 20 % slower)
#ifndef E5MA_CAST_NT_IN
#define E5MA_CAST_NT_IN 0
#endif
#ifndef E5MA_CAST_NT_OUT
#define E5MA_CAST_NT_OUT 1
#endif

template <int TI, int TO, bool VEC, bool AMAX>
__global__ __launch_bounds__(kThreads) void cast_kernel(const void *__restrict__ src, void *__restrict__ dst,
                                                        size_t count, const float *sinv_p, const float *qscale_p,
                                                        float *amax) {
  __shared__ float red[kThreads / 64];
  const float sinv = scale_or_one(sinv_p), qs = scale_or_one(qscale_p);
  const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x, stride = (size_t)gridDim.x * kThreads;
  float mx = 0.f;
  size_t tail = 0;
  if constexpr (VEC) {
    const size_t nvec = count / kVec;
    for (size_t c = tid; c < nvec; c += stride) {
      Pack<TI, kVec, E5MA_CAST_NT_IN> in;
      in.load(src, c * kVec);
      Pack<TO, kVec, E5MA_CAST_NT_OUT> out;
      float v[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        v[e] = in.get(e, sinv);
        if constexpr (AMAX) mx = amax_fold(mx, v[e]);
      }
      out.set(v, qs);
      out.store(dst, c * kVec);
    }
    tail = nvec * kVec;
  }
  for (size_t i = tail + tid; i < count; i += stride) {
    const float v = load_t<TI>(src, i, sinv);
    if constexpr (AMAX) mx = amax_fold(mx, v);
    store_t<TO>(dst, i, v, qs);
  }
  if constexpr (AMAX) amax_commit_block(amax, mx, red);
}

template <int TI, int TO>
hipError_t cast_to(const void *src, void *dst, size_t count, const float *sinv, const float *qs, float *amax,
                   int cap, hipStream_t s) {
  const bool vec = (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0;
  const size_t work = vec ? (count + kVec - 1) / kVec : count;
  const size_t blocks = (work + kThreads - 1) / kThreads;
  const int grid = (int)(blocks < (size_t)cap ? blocks : (size_t)cap);
#define E5MA_CAST_LAUNCH(V, A) \
  cast_kernel<TI, TO, V, A><<<grid, kThreads, 0, s>>>(src, dst, count, sinv, qs, amax)
  if (vec) {
    if (amax) E5MA_CAST_LAUNCH(true, true); else E5MA_CAST_LAUNCH(true, false);
  } else {
    if (amax) E5MA_CAST_LAUNCH(false, true); else E5MA_CAST_LAUNCH(false, false);
  }
#undef E5MA_CAST_LAUNCH
  return hipGetLastError();
}

template <int TI>
hipError_t cast_from(int tout, const void *src, void *dst, size_t count, const float *sinv, const float *qs,
                     float *amax, int cap, hipStream_t s) {
  switch (tout) {
    case E5MA_E5M2: return cast_to<TI, E5MA_E5M2>(src, dst, count, sinv, qs, amax, cap, s);
    case E5MA_E4M3: return cast_to<TI, E5MA_E4M3>(src, dst, count, sinv, qs, amax, cap, s);
    case E5MA_BF16: return cast_to<TI, E5MA_BF16>(src, dst, count, sinv, qs, amax, cap, s);
    case E5MA_FP16: return cast_to<TI, E5MA_FP16>(src, dst, count, sinv, qs, amax, cap, s);
    default: return cast_to<TI, E5MA_FP32>(src, dst, count, sinv, qs, amax, cap, s);
  }
}

}  // namespace

hipError_t launch_cast(int tin, int tout, const void *src, void *dst, size_t count, const float *sinv,
                       const float *qscale, float *amax, const Tuning &t, hipStream_t s) {
  const int cap = t.cast_grid > 0 ? t.cast_grid : 8192;
  switch (tin) {
    case E5MA_E5M2: return cast_from<E5MA_E5M2>(tout, src, dst, count, sinv, qscale, amax, cap, s);
    case E5MA_E4M3: return cast_from<E5MA_E4M3>(tout, src, dst, count, sinv, qscale, amax, cap, s);
    case E5MA_BF16: return cast_from<E5MA_BF16>(tout, src, dst, count, sinv, qscale, amax, cap, s);
    case E5MA_FP16: return cast_from<E5MA_FP16>(tout, src, dst, count, sinv, qscale, amax, cap, s);
    default: return cast_from<E5MA_FP32>(tout, src, dst, count, sinv, qscale, amax, cap, s);
  }
}

}  // namespace e5ma
