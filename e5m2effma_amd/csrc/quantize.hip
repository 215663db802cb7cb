// quantize.hip -- e5ma_quantize: FP8 codes with a scale taken from the data's own amax, the step the
// reference composes from torch operations and e5ma_cast in Float8Tensor.from_float
// (binds/python/e5m2effma/tensor.py:60-74):
//   amax = max |v| (NaN propagates), a = max(amax, 1e-12), scale = fl(fl(1 / a) * qmax),
//   codes = RNE satfinite of v * scale, scale_inv = 1 / scale          (v = src * src_scale_inv)
// torch evaluates `qmax / amax` as amax.reciprocal() * qmax, hence the two roundings.
//
// Per tensor, HBM-bound over two passes (in + in + out bytes per element):
//   q_amax_kernel  abs-max folded as integer maxima of |v|'s bit pattern (NaN patterns order above
//                  Inf, so a NaN is kept, as torch's amax keeps it), one atomicMax per block into the
//                  caller's scale_inv word, which a one-thread kernel has cleared first;
//   q_cast_kernel  every block derives the scale from that word and encodes, 16 elements per thread;
//   q_finish       replaces the word by scale_inv (and writes amax), after every block has read it.
// Per row: rows of at most 16384 elements (16-byte aligned, a multiple of 16) stay in one block's
// registers between the amax and the encoding, so HBM sees in + out bytes per element; longer or
// unaligned rows run one wave per row and are read a second time for the encoding.
#include "e5ma_host.hpp"
#include "vec.hpp"

// FP8 codes are stored non-temporally (written once, never read back by the library).  Measured on
// 8192^2 FP32: per tensor (amax pass + scaled cast) 108.1 -> 92.6 us, per row 64.7 -> 60.9 us.
#ifndef E5MA_QUANT_NT_OUT
#define E5MA_QUANT_NT_OUT 1
#endif

namespace e5ma {
namespace {

using namespace dev;
constexpr int kThreads = 256;
constexpr int kVec = 16;

__device__ __forceinline__ uint32_t abs_bits_max(uint32_t m, float v) {
  const uint32_t a = f2u(v) & 0x7FFFFFFFu;
  return a > m ? a : m;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t m) {
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    const uint32_t t = (uint32_t)__shfl_xor((int)m, o, 64);
    m = t > m ? t : m;
  }
  return m;
}
// torch's amax.clamp_min(1e-12) (a NaN stays NaN), then reciprocal() * qmax
__device__ __forceinline__ float quant_scale(uint32_t abits, float qmax) {
  const float a = abits > 0x7F800000u ? u2f(0x7FC00000u) : fmaxf(u2f(abits), 1e-12f);
  const float r = 1.0f / a;
  return r * qmax;
}

__global__ void q_clear_kernel(uint32_t *word) { *word = 0u; }

template <int TI, bool VEC>
__global__ __launch_bounds__(kThreads) void q_amax_kernel(const void *__restrict__ src, size_t count,
                                                          const float *sinv_p, uint32_t *word) {
  __shared__ uint32_t red[kThreads / 64];
  const float sinv = scale_or_one(sinv_p);
  const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x, stride = (size_t)gridDim.x * kThreads;
  uint32_t m = 0;
  size_t tail = 0;
  if constexpr (VEC) {
    const size_t nvec = count / kVec;
    for (size_t c = tid; c < nvec; c += stride) {
      Pack<TI, kVec> in;
      in.load(src, c * kVec);
#pragma unroll
      for (int e = 0; e < kVec; ++e) m = abs_bits_max(m, in.get(e, sinv));
    }
    tail = nvec * kVec;
  }
  for (size_t i = tail + tid; i < count; i += stride) m = abs_bits_max(m, load_t<TI>(src, i, sinv));
  m = wave_umax(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = red[w] > m ? red[w] : m;
    // most blocks' maxima do not exceed the value already there: skip their atomics (a stale read
    // only costs an atomic; atomicMax alone decides the result)
    if (m > __atomic_load_n(word, __ATOMIC_RELAXED)) atomicMax(word, m);
  }
}

template <int TI, int TO, bool VEC>
__global__ __launch_bounds__(kThreads) void q_cast_kernel(const void *__restrict__ src, void *__restrict__ dst,
                                                          size_t count, const float *sinv_p, const uint32_t *word,
                                                          float qmax) {
  const float sinv = scale_or_one(sinv_p), qs = quant_scale(*word, qmax);
  const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x, stride = (size_t)gridDim.x * kThreads;
  size_t tail = 0;
  if constexpr (VEC) {
    const size_t nvec = count / kVec;
    for (size_t c = tid; c < nvec; c += stride) {
      Pack<TI, kVec> in;
      in.load(src, c * kVec);
      Pack<TO, kVec, E5MA_QUANT_NT_OUT> out;
      float v[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = in.get(e, sinv);
      out.set(v, qs);
      out.store(dst, c * kVec);
    }
    tail = nvec * kVec;
  }
  for (size_t i = tail + tid; i < count; i += stride) store_t<TO>(dst, i, load_t<TI>(src, i, sinv), qs);
}

__global__ void q_finish_kernel(uint32_t *word, float *amax, float qmax) {
  const uint32_t ab = *word;
  const float s = quant_scale(ab, qmax);
  *(float *)word = 1.0f / s;
  if (amax) *amax = u2f(ab);
}

// one wave per row of cols elements (row r at element offset r * cols)
template <int TI, int TO, bool VEC>
__global__ __launch_bounds__(kThreads) void q_rows_kernel(const void *__restrict__ src, void *__restrict__ dst,
                                                          size_t rows, size_t cols, const float *sinv_p, float qmax,
                                                          float *scale_inv, float *amax) {
  const size_t row = (size_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves leave together: no barrier follows
  const int lane = threadIdx.x & 63;
  const float sinv = scale_or_one(sinv_p);
  const size_t base = row * cols;
  uint32_t m = 0;
  size_t tail = 0;
  if constexpr (VEC) {
    const size_t nvec = cols / kVec;
    for (size_t c = lane; c < nvec; c += 64) {
      Pack<TI, kVec> in;
      in.load(src, base + c * kVec);
#pragma unroll
      for (int e = 0; e < kVec; ++e) m = abs_bits_max(m, in.get(e, sinv));
    }
    tail = nvec * kVec;
  }
  for (size_t i = tail + lane; i < cols; i += 64) m = abs_bits_max(m, load_t<TI>(src, base + i, sinv));
  m = wave_umax(m);
  const float qs = quant_scale(m, qmax);
  if constexpr (VEC) {
    const size_t nvec = cols / kVec;
    for (size_t c = lane; c < nvec; c += 64) {
      Pack<TI, kVec> in;
      in.load(src, base + c * kVec);
      Pack<TO, kVec, E5MA_QUANT_NT_OUT> out;
      float v[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = in.get(e, sinv);
      out.set(v, qs);
      out.store(dst, base + c * kVec);
    }
  }
  for (size_t i = tail + lane; i < cols; i += 64) store_t<TO>(dst, base + i, load_t<TI>(src, base + i, sinv), qs);
  if (lane == 0) {
    scale_inv[row] = 1.0f / qs;
    if (amax) amax[row] = u2f(m);
  }
}

// One block per row, the row held in registers: thread t owns 16-element chunks t, t + kThreads, ...
// (CPL of them: rows of at most CPL * kThreads * kVec elements), block-wide amax through LDS.  With
// 2 chunks per thread an FP32 row of 8192 elements costs about 40 VGPRs, so 8 rows run per CU and
// 8192 rows take 4 even rounds (one wave per row, 151 VGPRs, took 2.7 rounds: 85 us against 63 us for
// the same bytes through the cast kernel).
template <int TI, int TO, int CPL>
__global__ __launch_bounds__(kThreads) void q_rows_blk_kernel(const void *__restrict__ src, void *__restrict__ dst,
                                                              size_t cols, const float *sinv_p, float qmax,
                                                              float *scale_inv, float *amax) {
  __shared__ uint32_t red[kThreads / 64];
  const size_t row = blockIdx.x;
  const int t = threadIdx.x;
  const float sinv = scale_or_one(sinv_p);
  const size_t base = row * cols;
  const int nvec = (int)(cols / kVec);
  Pack<TI, kVec> in[CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q)
    if (t + kThreads * q < nvec) in[q].load(src, base + (size_t)(t + kThreads * q) * kVec);
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < CPL; ++q)
    if (t + kThreads * q < nvec) {
#pragma unroll
      for (int e = 0; e < kVec; ++e) m = abs_bits_max(m, in[q].get(e, sinv));
    }
  m = wave_umax(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) m = red[w] > m ? red[w] : m;
  const float qs = quant_scale(m, qmax);
#pragma unroll
  for (int q = 0; q < CPL; ++q)
    if (t + kThreads * q < nvec) {
      Pack<TO, kVec, E5MA_QUANT_NT_OUT> out;
      float v[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[e] = in[q].get(e, sinv);
      out.set(v, qs);
      out.store(dst, base + (size_t)(t + kThreads * q) * kVec);
    }
  if (t == 0) {
    scale_inv[row] = 1.0f / qs;
    if (amax) amax[row] = u2f(m);
  }
}

template <int TI, int TO>
hipError_t quantize_to(const void *src, void *dst, size_t rows, size_t cols, const float *sinv, float qmax,
                       bool per_row, float *scale_inv, float *amax, int amax_cap, int cast_cap, hipStream_t s) {
  if (per_row) {
    const bool vec = cols % kVec == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0;
    const size_t blocks = (rows + kThreads / 64 - 1) / (kThreads / 64);
    constexpr size_t kBlkRow = (size_t)kThreads * kVec;  // elements per chunk round of a block
    if (vec && cols <= 2 * kBlkRow)
      q_rows_blk_kernel<TI, TO, 2><<<rows, kThreads, 0, s>>>(src, dst, cols, sinv, qmax, scale_inv, amax);
    else if (vec && cols <= 4 * kBlkRow)
      q_rows_blk_kernel<TI, TO, 4><<<rows, kThreads, 0, s>>>(src, dst, cols, sinv, qmax, scale_inv, amax);
    else if (vec) q_rows_kernel<TI, TO, true><<<blocks, kThreads, 0, s>>>(src, dst, rows, cols, sinv, qmax, scale_inv, amax);
    else q_rows_kernel<TI, TO, false><<<blocks, kThreads, 0, s>>>(src, dst, rows, cols, sinv, qmax, scale_inv, amax);
    return hipGetLastError();
  }
  const size_t count = rows * cols;
  const bool vec = (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0;
  const size_t work = vec ? (count + kVec - 1) / kVec : count;
  const size_t blocks = (work + kThreads - 1) / kThreads;
  // the read-only amax pass and the scaled cast measured fastest with different grid caps
  const int ga = (int)(blocks < (size_t)amax_cap ? blocks : (size_t)amax_cap);
  const int gc = (int)(blocks < (size_t)cast_cap ? blocks : (size_t)cast_cap);
  uint32_t *word = (uint32_t *)scale_inv;
  q_clear_kernel<<<1, 1, 0, s>>>(word);
  if (vec) {
    q_amax_kernel<TI, true><<<ga, kThreads, 0, s>>>(src, count, sinv, word);
    q_cast_kernel<TI, TO, true><<<gc, kThreads, 0, s>>>(src, dst, count, sinv, word, qmax);
  } else {
    q_amax_kernel<TI, false><<<ga, kThreads, 0, s>>>(src, count, sinv, word);
    q_cast_kernel<TI, TO, false><<<gc, kThreads, 0, s>>>(src, dst, count, sinv, word, qmax);
  }
  q_finish_kernel<<<1, 1, 0, s>>>(word, amax, qmax);
  return hipGetLastError();
}

template <int TI>
hipError_t quantize_from(int tout, const void *src, void *dst, size_t rows, size_t cols, const float *sinv,
                         float qmax, bool per_row, float *scale_inv, float *amax, int ca, int cc, hipStream_t s) {
  if (tout == E5MA_E5M2) return quantize_to<TI, E5MA_E5M2>(src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
  return quantize_to<TI, E5MA_E4M3>(src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
}

}  // namespace

hipError_t launch_quantize(int tin, int tout, const void *src, void *dst, size_t rows, size_t cols, const float *sinv,
                           float qmax, bool per_row, float *scale_inv, float *amax, const Tuning &t, hipStream_t s) {
  const int ca = t.quant_grid > 0 ? t.quant_grid : 8192, cc = t.cast_grid > 0 ? t.cast_grid : 8192;
  switch (tin) {
    case E5MA_E5M2: return quantize_from<E5MA_E5M2>(tout, src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
    case E5MA_E4M3: return quantize_from<E5MA_E4M3>(tout, src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
    case E5MA_BF16: return quantize_from<E5MA_BF16>(tout, src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
    case E5MA_FP16: return quantize_from<E5MA_FP16>(tout, src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
    default: return quantize_from<E5MA_FP32>(tout, src, dst, rows, cols, sinv, qmax, per_row, scale_inv, amax, ca, cc, s);
  }
}

}  // namespace e5ma
