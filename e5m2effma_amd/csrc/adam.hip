// adam.hip -- e5ma_adam: fused in-place Adam / AdamW step over FP32 or BF16 state, with an optional
// E4M3 / E5M2 copy of the updated weights and its amax (reference src/adamw_e5m2effma.cu:11-120).
// HBM-bound streaming kernel: 8 elements per thread per step through 16-byte accesses when every
// buffer is aligned for them; element by element otherwise.  Both paths compute each element with
// adam_elem, so results do not depend on alignment.
#include "e5ma_host.hpp"
#include "vec.hpp"

namespace e5ma {
namespace {

using namespace dev;
constexpr int kThreads = 256;
constexpr int kVec = 8;
constexpr int kNoCopy = -1;
// launch shape: non-temporal accesses per state width (measured on 2^28 parameters: BF16 states
// 5.16 TB/s with non-temporal accesses and 65536 blocks; FP32 states 4.93 TB/s with ordinary accesses
// and 8192 blocks, where non-temporal accesses cost 15%); the grid caps come from the device's Tuning
#ifndef E5MA_ADAM_NT_BF16
#define E5MA_ADAM_NT_BF16 1
#endif
#ifndef E5MA_ADAM_NT_FP32
#define E5MA_ADAM_NT_FP32 0
#endif

// One element in the documented order (include/e5m2effma.h:88-94; reference
// src/adamw_e5m2effma.cu:17-25).  Division and square root are correctly rounded (the library is
// built with -fhip-fp32-correctly-rounded-divide-sqrt and without fast-math); nothing is contracted.
// The mode flag, not the coefficient's value, selects the weight-decay term: fma(0, p, g) is not g when
// p is Inf or NaN.
__device__ __forceinline__ void adam_elem(const AdamCoefficients &a, float g, float &p, float &m, float &v) {
  g = g * a.grad_mul;
  if (!a.decoupled) g = __builtin_fmaf(a.l2, p, g);
  m = __builtin_fmaf(a.b1, m, a.c1 * g);
  v = __builtin_fmaf(a.b2, v, a.c2 * (g * g));
  const float u = (m * a.corr1) / (__builtin_sqrtf(v * a.corr2) + a.eps);
  if (a.decoupled) p = __builtin_fmaf(-a.decay, p, p);
  p = __builtin_fmaf(-a.lr, u, p);
}

template <int PT, int GT, int MT, int QT, bool VEC>
__global__ __launch_bounds__(kThreads) void adam_kernel(AdamCoefficients a, size_t count, void *__restrict__ p_,
                                                        const void *__restrict__ g_, void *__restrict__ m_,
                                                        void *__restrict__ v_, uint8_t *__restrict__ q_,
                                                        const float *qscale_p, float *amax) {
  __shared__ float red[kThreads / 64];
  constexpr bool kCopy = QT != kNoCopy;
  const float qs = kCopy ? scale_or_one(qscale_p) : 1.f;
  const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x, stride = (size_t)gridDim.x * kThreads;
  float mx = 0.f;
  size_t tail = 0;
  if constexpr (VEC) {
    const size_t nvec = count / kVec;
    for (size_t c = tid; c < nvec; c += stride) {
      const size_t i = c * kVec;
      constexpr bool kNT = PT == E5MA_FP32 ? E5MA_ADAM_NT_FP32 : E5MA_ADAM_NT_BF16;
      Pack<GT, kVec, kNT> G;
      Pack<PT, kVec, kNT> P;
      Pack<MT, kVec, kNT> M, V;
      G.load(g_, i);
      P.load(p_, i);
      M.load(m_, i);
      V.load(v_, i);
      Pack<PT, kVec, kNT> Po;
      Pack<MT, kVec, kNT> Mo, Vo;
      Po.clear();
      Mo.clear();
      Vo.clear();
      uint32_t q[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        float p = P.get(e, 1.f), m = M.get(e, 1.f), v = V.get(e, 1.f);
        adam_elem(a, G.get(e, 1.f), p, m, v);
        Po.put(e, p, 1.f);
        Mo.put(e, m, 1.f);
        Vo.put(e, v, 1.f);
        if constexpr (kCopy) {
          q[e >> 2] |= f32_to_fp8t<QT>(p * qs) << (8 * (e & 3));
          mx = amax_fold(mx, p);
        }
      }
      Po.store(p_, i);
      Mo.store(m_, i);
      Vo.store(v_, i);
      if constexpr (kCopy) *(uint2 *)(q_ + i) = make_uint2(q[0], q[1]);
    }
    tail = nvec * kVec;
  }
  for (size_t i = tail + tid; i < count; i += stride) {
    float p = load_t<PT>(p_, i, 1.f), m = load_t<MT>(m_, i, 1.f), v = load_t<MT>(v_, i, 1.f);
    adam_elem(a, load_t<GT>(g_, i, 1.f), p, m, v);
    store_t<PT>(p_, i, p, 1.f);
    store_t<MT>(m_, i, m, 1.f);
    store_t<MT>(v_, i, v, 1.f);
    if constexpr (kCopy) {
      q_[i] = (uint8_t)f32_to_fp8t<QT>(p * qs);
      mx = amax_fold(mx, p);
    }
  }
  if constexpr (kCopy) {
    if (amax) amax_commit_block(amax, mx, red);
  }
}

template <int PT, int GT, int MT, int QT>
hipError_t adam_v(const AdamCoefficients &a, size_t count, void *p, const void *g, void *m, void *v, uint8_t *q,
                  const float *qs, float *amax, int cap, hipStream_t s) {
  const auto a16 = [](const void *x) { return ((uintptr_t)x & 15u) == 0; };
  const bool vec = a16(p) && a16(g) && a16(m) && a16(v) && ((uintptr_t)q & 7u) == 0;
  const size_t work = vec ? (count + kVec - 1) / kVec : count;
  const size_t blocks = (work + kThreads - 1) / kThreads;
  const int grid = (int)(blocks < (size_t)cap ? blocks : (size_t)cap);
  if (vec) adam_kernel<PT, GT, MT, QT, true><<<grid, kThreads, 0, s>>>(a, count, p, g, m, v, q, qs, amax);
  else adam_kernel<PT, GT, MT, QT, false><<<grid, kThreads, 0, s>>>(a, count, p, g, m, v, q, qs, amax);
  return hipGetLastError();
}

template <int PT, int GT, int MT>
hipError_t adam_q(int qt, const AdamCoefficients &a, size_t count, void *p, const void *g, void *m, void *v, uint8_t *q,
                  const float *qs, float *amax, int cap, hipStream_t s) {
  if (!q) return adam_v<PT, GT, MT, kNoCopy>(a, count, p, g, m, v, q, qs, amax, cap, s);
  if (qt == E5MA_E5M2) return adam_v<PT, GT, MT, E5MA_E5M2>(a, count, p, g, m, v, q, qs, amax, cap, s);
  return adam_v<PT, GT, MT, E5MA_E4M3>(a, count, p, g, m, v, q, qs, amax, cap, s);
}

template <int PT, int GT>
hipError_t adam_m(int mt, int qt, const AdamCoefficients &a, size_t count, void *p, const void *g, void *m, void *v,
                  uint8_t *q, const float *qs, float *amax, int cap, hipStream_t s) {
  if (mt == E5MA_BF16) return adam_q<PT, GT, E5MA_BF16>(qt, a, count, p, g, m, v, q, qs, amax, cap, s);
  return adam_q<PT, GT, E5MA_FP32>(qt, a, count, p, g, m, v, q, qs, amax, cap, s);
}

template <int PT>
hipError_t adam_g(int gt, int mt, int qt, const AdamCoefficients &a, size_t count, void *p, const void *g, void *m,
                  void *v, uint8_t *q, const float *qs, float *amax, int cap, hipStream_t s) {
  if (gt == E5MA_BF16) return adam_m<PT, E5MA_BF16>(mt, qt, a, count, p, g, m, v, q, qs, amax, cap, s);
  if (gt == E5MA_FP16) return adam_m<PT, E5MA_FP16>(mt, qt, a, count, p, g, m, v, q, qs, amax, cap, s);
  return adam_m<PT, E5MA_FP32>(mt, qt, a, count, p, g, m, v, q, qs, amax, cap, s);
}

}  // namespace

hipError_t launch_adam(const AdamCoefficients &a, size_t count, int pt, void *p, int gt, const void *g, int mt, void *m,
                       void *v, int qt, uint8_t *q, const float *qscale, float *amax, const Tuning &t,
                       hipStream_t s) {
  const int cap = pt == E5MA_BF16 ? t.adam_grid_bf16 : t.adam_grid_fp32;
  if (pt == E5MA_BF16) return adam_g<E5MA_BF16>(gt, mt, qt, a, count, p, g, m, v, q, qscale, amax, cap > 0 ? cap : 65536, s);
  return adam_g<E5MA_FP32>(gt, mt, qt, a, count, p, g, m, v, q, qscale, amax, cap > 0 ? cap : 8192, s);
}

}  // namespace e5ma
