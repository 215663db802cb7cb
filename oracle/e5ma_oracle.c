/* e5ma_oracle.c -- CPU restatement of the reference's FP8 compute semantics (test infrastructure).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, as the
 * checker or as the timed CPU baseline; the product library never does.  Compiled with
 * -O2 -ffp-contract=off -mfma (fmaf is a single fused multiply-add, every other float operation
 * rounds once, as written).  Reference paths are relative to /root/reference.
 */
#include "e5ma_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline int is_fp8(int t) { return t == ORC_E4M3 || t == ORC_E5M2; }

/* ---------------------------------------------------------------------------------------------
 * Decoders
 * ------------------------------------------------------------------------------------------- */

/* Exact value of an E4M3 (OCP "fn") code; the NaN code (S.1111.111) decodes to NaN.
 * Follows src/e5m2effma.cuh:54-58 and tests/test_util.h:21-25. */
float orc_e4m3_value(uint8_t b) {
  const int e = (b >> 3) & 15, f = b & 7;
  if ((b & 0x7F) == 0x7F) return NAN;
  const float v = e ? ldexpf((float)(8 + f), e - 10) : ldexpf((float)f, -9);
  return (b & 0x80) ? -v : v;
}

/* Exact value of an E5M2 code (the upper byte of an IEEE binary16), Inf / NaN included.
 * Follows src/e5m2effma.cuh:69-72 and tests/test_util.h:26-30. */
float orc_e5m2_value(uint8_t b) {
  const int e = (b >> 2) & 31, f = b & 3;
  float v;
  if (e == 31) {
    if (f) return NAN;
    v = INFINITY;
  } else {
    v = e ? ldexpf((float)(4 + f), e - 17) : ldexpf((float)f, -16);
  }
  return (b & 0x80) ? -v : v;
}

/* The reference's GEMM-operand decode: the exponent/mantissa formula applied to every code, so the
 * out-of-contract E4M3 NaN code reads as 480 and the E5M2 Inf / NaN codes as 65536..114688.
 * Follows src/e5m2effma.cuh:43-52 and :59-68 (the bit-shift decode times 2^120 / 2^112). */
float orc_e4m3_operand(uint8_t b) {
  const int e = (b >> 3) & 15, f = b & 7;
  const float v = e ? ldexpf((float)(8 + f), e - 10) : ldexpf((float)f, -9);
  return (b & 0x80) ? -v : v;
}
float orc_e5m2_operand(uint8_t b) {
  const int e = (b >> 2) & 31, f = b & 3;
  const float v = e ? ldexpf((float)(4 + f), e - 17) : ldexpf((float)f, -16);
  return (b & 0x80) ? -v : v;
}

/* BF16 is the upper half of an FP32 (src/e5m2effma.cuh:140). */
float orc_bf16_value(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE-754 binary16 value (the reference uses cuda_fp16's __half2float, src/e5m2effma.cuh:141). */
float orc_f16_value(uint16_t h) {
  const int e = (h >> 10) & 31, f = h & 1023;
  float v;
  if (e == 31) {
    if (f) return NAN;
    v = INFINITY;
  } else {
    v = e ? ldexpf((float)(1024 + f), e - 25) : ldexpf((float)f, -24);
  }
  return (h & 0x8000) ? -v : v;
}

/* ---------------------------------------------------------------------------------------------
 * Encoders
 * ------------------------------------------------------------------------------------------- */

/* FP32 -> BF16 bits, round to nearest even on the dropped 16 bits; every NaN -> 0x7FC0.
 * Follows src/e5m2effma.cuh:80-88 (and the remainder formulation of tests/test_e5m2effma.cu:82-94). */
uint16_t orc_f32_to_bf16(float x) {
  const uint32_t u = f2u(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  uint32_t hi = u >> 16;
  const uint32_t lo = u & 0xFFFFu;
  if (lo > 0x8000u || (lo == 0x8000u && (hi & 1u))) ++hi;
  return (uint16_t)hi;
}

/* FP32 -> IEEE binary16, round to nearest even, overflow to Inf (the reference uses cuda_fp16's
 * __float2half_rn, src/e5m2effma.cuh:150).  NaN -> a quiet NaN (its bits are not part of the
 * contract). */
uint16_t orc_f32_to_f16(float x) {
  const uint32_t u = f2u(x), s = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7E00;
  if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u); /* >= 65520 rounds to Inf */
  if (a >= 0x38800000u) {                                /* >= 2^-14: normal binary16 */
    const uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);
    return (uint16_t)(s | ((r >> 13) - (112u << 10)));
  }
  /* subnormal grid 2^-24; the scaling by 2^24 is exact, nearbyintf rounds half to even */
  const float q = nearbyintf(u2f(a) * 16777216.0f);
  return (uint16_t)(s | (uint32_t)q);
}

/* FP32 -> FP8 with `mbits` mantissa bits and exponent bias `bias`: round to nearest even;
 * |x| >= the largest finite value (Inf included) saturates to it; every NaN -> 0x7F (sign dropped).
 * Restates src/e5m2effma.cuh:90-124 (cvt.rn.satfinite semantics). */
static uint8_t fp8_encode(float x, int mbits, int bias, uint32_t max_bits, uint8_t max_code) {
  const uint32_t u = f2u(x), s = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7F;
  if (a >= max_bits) return (uint8_t)(s | max_code);
  const uint32_t min_normal = (uint32_t)(128 - bias) << 23;
  if (a < min_normal) { /* subnormal grid 2^(1 - bias - mbits); the scaling is exact */
    const float q = nearbyintf(ldexpf(u2f(a), bias - 1 + mbits));
    return (uint8_t)(s | (uint32_t)q);
  }
  const int drop = 23 - mbits;
  const uint32_t r = a + ((1u << (drop - 1)) - 1u) + ((a >> drop) & 1u);
  return (uint8_t)(s | ((r >> drop) - ((uint32_t)(127 - bias) << mbits)));
}
uint8_t orc_f32_to_e4m3(float x) { return fp8_encode(x, 3, 7, 0x43E00000u, 0x7E); }
uint8_t orc_f32_to_e5m2(float x) { return fp8_encode(x, 2, 15, 0x47600000u, 0x7B); }

/* Independent FP32 -> FP8 encoder for self-checks: locate |x| among the finite code values by
 * binary search and round by comparing with the exact midpoint (ties to the even code).  The same
 * specification as the reference's encoder test (tests/test_e5m2effma.cu:96-124), stated afresh. */
uint8_t orc_fp8_encode_search(float x, int fmt) {
  const int top = fmt == ORC_E5M2 ? 0x7B : 0x7E;
  const uint32_t s = (f2u(x) >> 24) & 0x80u;
  const double a = fabs((double)x);
  if (x != x) return 0x7F;
  const double vmax = fmt == ORC_E5M2 ? 57344.0 : 448.0;
  if (a >= vmax) return (uint8_t)(s | (uint32_t)top);
  int lo = 0, hi = top; /* value(lo) <= a < value(hi) */
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    const double v = fmt == ORC_E5M2 ? orc_e5m2_value((uint8_t)mid) : orc_e4m3_value((uint8_t)mid);
    if (v <= a) lo = mid; else hi = mid;
  }
  const double vl = fmt == ORC_E5M2 ? orc_e5m2_value((uint8_t)lo) : orc_e4m3_value((uint8_t)lo);
  const double vh = fmt == ORC_E5M2 ? orc_e5m2_value((uint8_t)hi) : orc_e4m3_value((uint8_t)hi);
  const double midv = 0.5 * (vl + vh);
  int c;
  if (a == vl) c = lo;
  else if (a < midv) c = lo;
  else if (a > midv) c = hi;
  else c = (lo & 1) ? hi : lo;
  return (uint8_t)(s | (uint32_t)c);
}

size_t orc_encode_selfcheck(int fmt, uint64_t start, uint64_t stop, uint64_t step, uint32_t *first_bad) {
  size_t bad = 0;
  for (uint64_t k = start; k < stop; k += step) {
    const float x = u2f((uint32_t)k);
    const uint8_t got = fmt == ORC_E5M2 ? orc_f32_to_e5m2(x) : orc_f32_to_e4m3(x);
    if (got != orc_fp8_encode_search(x, fmt)) {
      if (!bad && first_bad) *first_bad = (uint32_t)k;
      ++bad;
    }
  }
  return bad;
}

/* ---------------------------------------------------------------------------------------------
 * Typed element access (src/e5m2effma.cuh:131-153)
 * ------------------------------------------------------------------------------------------- */
float orc_load(int t, const void *p, size_t i, float sinv) {
  switch (t) {
    case ORC_E5M2: return orc_e5m2_value(((const uint8_t *)p)[i]) * sinv;
    case ORC_E4M3: return orc_e4m3_value(((const uint8_t *)p)[i]) * sinv;
    case ORC_BF16: return orc_bf16_value(((const uint16_t *)p)[i]);
    case ORC_FP16: return orc_f16_value(((const uint16_t *)p)[i]);
    default: return ((const float *)p)[i];
  }
}
void orc_store(int t, void *p, size_t i, float v, float qscale) {
  switch (t) {
    case ORC_E5M2: ((uint8_t *)p)[i] = orc_f32_to_e5m2(v * qscale); break;
    case ORC_E4M3: ((uint8_t *)p)[i] = orc_f32_to_e4m3(v * qscale); break;
    case ORC_BF16: ((uint16_t *)p)[i] = orc_f32_to_bf16(v); break;
    case ORC_FP16: ((uint16_t *)p)[i] = orc_f32_to_f16(v); break;
    default: ((float *)p)[i] = v;
  }
}

void orc_encode_batch(int t, const float *x, void *out, size_t n, float qscale) {
  for (size_t i = 0; i < n; ++i) orc_store(t, out, i, x[i], qscale);
}
void orc_decode_batch(int t, const void *p, float *out, size_t n, float sinv) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_load(t, p, i, sinv);
}

/* |v| folded into a running maximum; every NaN (quiet or signalling) is ignored, as the reference's
 * device reduction ignores it (src/e5m2effma.cuh:192, fmaxf on the GPU returns the non-NaN operand).
 * glibc's fmaxf is not used: it returns NaN for a signalling-NaN operand. */
static inline float amax_fold(float m, float v) {
  const float a = fabsf(v);
  return a > m ? a : m;
}

/* amax commit of the reference: |v| max-reduced with fmaxf (NaN ignored), then an integer atomicMax
 * of the float bits into *amax, issued only for a positive partial maximum
 * (src/e5m2effma.cuh:190-195). */
static float amax_merge(float amax_in, float m) {
  if (!(m > 0.f)) return amax_in;
  return (int32_t)f2u(m) > (int32_t)f2u(amax_in) ? m : amax_in;
}

/* ---------------------------------------------------------------------------------------------
 * One MAC of the exact model: RN_BF16(acc + a*b) for FP8 a, b (fa, fb: 0 = E4M3, 1 = E5M2, the
 * reference's e5ma_ref enum) and a BF16 accumulator.  Restates tests/e5m2effma_ref.h:114-129.
 * The FP8 product is exact in double; acc + product is rounded to double, then to FP32, then to
 * BF16: each intermediate precision is at least 2p + 2 bits of the next one for sums of two
 * 8-bit-significand values, so the chain equals a single rounding of the exact sum (pinned against
 * the reference model by tests/test_oracle_lane.py).
 * ------------------------------------------------------------------------------------------- */
uint16_t orc_lane(uint8_t a, uint8_t b, uint16_t acc, int fa, int fb) {
  const int sa = fa ? (a & 0x7C) == 0x7C : (a & 0x7F) == 0x7F;
  const int sb = fb ? (b & 0x7C) == 0x7C : (b & 0x7F) == 0x7F;
  if (sa || sb) return 0x7FC0;
  if ((acc & 0x7FFF) > 0x7F80) return 0x7FC0;
  if ((acc & 0x7FFF) == 0x7F80) return acc;
  const double pa = fa ? orc_e5m2_value(a) : orc_e4m3_value(a);
  const double pb = fb ? orc_e5m2_value(b) : orc_e4m3_value(b);
  const double sum = (double)orc_bf16_value(acc) + pa * pb;
  return orc_f32_to_bf16((float)sum);
}

void orc_lane_batch(const uint8_t *a, const uint8_t *b, const uint16_t *acc, int fa, int fb,
                    uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_lane(a[i], b[i], acc[i], fa, fb);
}

size_t orc_lane_compare(orc_ref_lane_fn ref, const uint16_t *accs, size_t nacc, int fa, int fb,
                        uint32_t *first_bad) {
  size_t bad = 0;
  for (size_t c = 0; c < nacc; ++c)
    for (uint32_t a = 0; a < 256; ++a)
      for (uint32_t b = 0; b < 256; ++b) {
        const uint32_t r = ref(a, b, accs[c], fa, fb);
        if (r != orc_lane((uint8_t)a, (uint8_t)b, accs[c], fa, fb)) {
          if (!bad && first_bad) *first_bad = (uint32_t)accs[c] << 16 | a << 8 | b;
          ++bad;
        }
      }
  return bad;
}

/* Outputs of any lane function (e.g. the reference model's ref_lane) over every FP8 pair (a, b) for
 * each accumulator in accs: out[(c * 256 + a) * 256 + b]. */
void orc_lane_sweep(orc_ref_lane_fn fn, const uint16_t *accs, size_t nacc, int fa, int fb,
                    uint16_t *out) {
  for (size_t c = 0; c < nacc; ++c)
    for (uint32_t a = 0; a < 256; ++a)
      for (uint32_t b = 0; b < 256; ++b)
        out[(c * 256 + a) * 256 + b] =
            fn ? (uint16_t)fn(a, b, accs[c], fa, fb) : orc_lane((uint8_t)a, (uint8_t)b, accs[c], fa, fb);
}

/* BASELINE config 1's CPU path: a row-major M x K by K x N product of FP8 codes as a chain of the
 * reference's MAC model over k (tests/e5m2effma_ref.h:114-129): out[i][j] = lane(a[i][K-1], b[K-1][j],
 * ... lane(a[i][0], b[0][j], +0)), a BF16 accumulator rounded once per MAC.  fn: the reference's own
 * ref_lane (compiled from its sources into _ref/libref.so) or NULL for the restatement above.  Rows
 * row0 .. row1 - 1 of out (BF16 bits). */
void orc_lane_gemm(orc_ref_lane_fn fn, const uint8_t *a, const uint8_t *b, int N, int K, int fa, int fb,
                   uint16_t *out, int row0, int row1) {
  for (int i = row0; i < row1; ++i)
    for (int j = 0; j < N; ++j) {
      uint16_t acc = 0;
      for (int k = 0; k < K; ++k) {
        const uint8_t x = a[(size_t)i * K + k], y = b[(size_t)k * N + j];
        acc = fn ? (uint16_t)fn(x, y, acc, fa, fb) : orc_lane(x, y, acc, fa, fb);
      }
      out[(size_t)i * N + j] = acc;
    }
}

/* ---------------------------------------------------------------------------------------------
 * e5ma_cast (src/e5m2effma.cu:53-63, 85-101): v = load(src) * sinv; amax = max |v|;
 * dst = store(v, qscale).  Returns the updated amax.
 * ------------------------------------------------------------------------------------------- */
float orc_cast(int tin, int tout, const void *src, void *dst, size_t count, float sinv,
               float qscale, float amax_in) {
  float m = 0.f;
  for (size_t i = 0; i < count; ++i) {
    const float v = orc_load(tin, src, i, sinv);
    m = amax_fold(m, v);
    orc_store(tout, dst, i, v, qscale);
  }
  return amax_merge(amax_in, m);
}

/* ---------------------------------------------------------------------------------------------
 * e5ma_gemm semantics (include/e5m2effma.h:6-31; src/gemm_e5m2effma.cu:194-208;
 * src/e5m2effma.cuh:209-241; host emulation tests/test_util.h:111-144)
 * ------------------------------------------------------------------------------------------- */
static float operand(int t, const void *p, size_t idx, int ocp) {
  switch (t) {
    case ORC_E5M2: {
      const uint8_t b = ((const uint8_t *)p)[idx];
      return ocp ? orc_e5m2_value(b) : orc_e5m2_operand(b);
    }
    case ORC_E4M3: {
      const uint8_t b = ((const uint8_t *)p)[idx];
      return ocp ? orc_e4m3_value(b) : orc_e4m3_operand(b);
    }
    case ORC_BF16: return orc_bf16_value(((const uint16_t *)p)[idx]);
    default: return ((const float *)p)[idx];
  }
}
static inline float opA(const orc_gemm_args *g, int i, int kk) {
  const size_t idx = g->transa ? (size_t)i * g->lda + kk : (size_t)kk * g->lda + i;
  return operand(g->adt, g->A, idx, g->ocp_operands);
}
static inline float opB(const orc_gemm_args *g, int kk, int j) {
  const size_t idx = g->transb ? (size_t)kk * g->ldb + j : (size_t)j * g->ldb + kk;
  return operand(g->bdt, g->B, idx, g->ocp_operands);
}
/* (alpha * sa[i]) * sb[j]; scale_inv only for FP8 operands (src/e5m2effma.cuh:209-222) */
static inline float out_scale(const orc_gemm_args *g, int i, int j) {
  float a = 1.f, b = 1.f;
  if (is_fp8(g->adt) && g->sa) a = g->sa_vec ? g->sa[i] : g->sa[0];
  if (is_fp8(g->bdt) && g->sb) b = g->sb_vec ? g->sb[j] : g->sb[0];
  return (g->alpha * a) * b;
}
static inline int c_dtype(const orc_gemm_args *g) { return g->C ? g->cdt : g->ddt; }
static inline int c_ld(const orc_gemm_args *g) { return g->C ? g->ldc : g->ldd; }

/* v = acc * s; v = v + bias[i]; v = fma(beta, cval, v) -- src/e5m2effma.cuh:224-233 */
float orc_epilogue(const orc_gemm_args *g, int i, int j, float acc, float cval) {
  float v = acc * out_scale(g, i, j);
  if (g->bias) v = v + orc_load(g->biasdt, g->bias, (size_t)i, 1.f);
  if (g->beta != 0.f) v = fmaf(g->beta, cval, v);
  return v;
}
static inline float c_value(const orc_gemm_args *g, const void *Cp, int i, int j) {
  if (g->beta == 0.f) return 0.f;
  return orc_load(c_dtype(g), Cp, (size_t)j * c_ld(g) + i, g->csinv);
}

typedef struct {
  const orc_gemm_args *g;
  int row0, row1, j0, j1;
  float amax;
} chain_job;

/* ascending-k fmaf chain per output (tests/test_util.h:122-123), columns [j0, j1) */
static void *chain_worker(void *arg) {
  chain_job *job = (chain_job *)arg;
  const orc_gemm_args *g = job->g;
  const int k = g->k;
  float *arow = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
  float *bcol = (float *)calloc((size_t)(k > 0 ? k : 1) * 8, sizeof(float));
  const void *Cp = g->C ? g->C : g->D;
  float m = 0.f;
  for (int j0 = job->j0; j0 < job->j1; j0 += 8) {
    const int nj = job->j1 - j0 < 8 ? job->j1 - j0 : 8;
    for (int jj = 0; jj < nj; ++jj)
      for (int kk = 0; kk < k; ++kk) bcol[(size_t)jj * k + kk] = opB(g, kk, j0 + jj);
    for (int i = job->row0; i < job->row1; ++i) {
      for (int kk = 0; kk < k; ++kk) arow[kk] = opA(g, i, kk);
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int kk = 0; kk < k; ++kk) {
        const float a = arow[kk];
        for (int jj = 0; jj < 8; ++jj) acc[jj] = fmaf(a, bcol[(size_t)jj * k + kk], acc[jj]);
      }
      for (int jj = 0; jj < nj; ++jj) {
        const int j = j0 + jj;
        const float v = orc_epilogue(g, i, j, acc[jj], c_value(g, Cp, i, j));
        m = amax_fold(m, v);
        orc_store(g->ddt, g->D, (size_t)j * g->ldd + i, v, g->qscale);
      }
    }
  }
  free(arow);
  free(bcol);
  job->amax = m;
  return NULL;
}

/* D rows [row0, row1) of the GEMM with the reference tiled kernel's ascending-k FFMA chain, over
 * nthreads POSIX threads: columns in groups of 8 split between them, or rows when there are fewer
 * groups than threads (a GEMV).  Each output's chain is the same either way.  Returns the updated amax. */
float orc_gemm_chain(const orc_gemm_args *g, float amax_in, int row0, int row1, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  if (row1 > g->m) row1 = g->m;
  if (row0 >= row1 || g->n <= 0) return amax_in;
  chain_job jobs[256];
  pthread_t th[256];
  int used = 0;
  if ((g->n + 7) / 8 >= nthreads) {
    const int per = ((g->n + nthreads - 1) / nthreads + 7) / 8 * 8;
    for (int t = 0; t < nthreads; ++t) {
      const int j0 = t * per, j1 = j0 + per < g->n ? j0 + per : g->n;
      if (j0 >= j1) break;
      jobs[used++] = (chain_job){g, row0, row1, j0, j1, 0.f};
    }
  } else {
    const int rows = row1 - row0, per = (rows + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; ++t) {
      const int r0 = row0 + t * per, r1 = r0 + per < row1 ? r0 + per : row1;
      if (r0 >= r1) break;
      jobs[used++] = (chain_job){g, r0, r1, 0, g->n, 0.f};
    }
  }
  for (int t = 1; t < used; ++t) pthread_create(&th[t], NULL, chain_worker, &jobs[t]);
  if (used) chain_worker(&jobs[0]);
  for (int t = 1; t < used; ++t) pthread_join(th[t], NULL);
  float m = 0.f;
  for (int t = 0; t < used; ++t) m = fmaxf(m, jobs[t].amax);
  return amax_merge(amax_in, m);
}

/* Exact-product dot products in double for sampled outputs: exact[s] = sum_k a*b (each FP8 / BF16
 * / FP32 product is exact in double; the double sum adds at most k * 2^-53 * mag), mag[s] =
 * sum_k |a*b|.  Operands as the matrix cores read them when ocp_operands is set. */
void orc_gemm_exact(const orc_gemm_args *g, const int *is, const int *js, size_t count,
                    double *exact, double *mag) {
  for (size_t s = 0; s < count; ++s) {
    double e = 0.0, a = 0.0;
    for (int kk = 0; kk < g->k; ++kk) {
      const double p = (double)opA(g, is[s], kk) * (double)opB(g, kk, js[s]);
      e += p;
      a += fabs(p);
    }
    exact[s] = e;
    mag[s] = a;
  }
}

static float round_down(double x) {
  float f = (float)x;
  if ((double)f > x) f = nextafterf(f, -INFINITY);
  return f;
}
static float round_up(double x) {
  float f = (float)x;
  if ((double)f < x) f = nextafterf(f, INFINITY);
  return f;
}
static int same_nan_or_equal(float a, float b) { return (a != a && b != b) || a == b; }

/* Checks sampled outputs of a GEMM against the bound |acc - exact| <= err_factor * k * 2^-24 * mag
 * (+ the double-sum error).  The epilogue is monotone in acc, so the stored output must lie between
 * the outputs the epilogue produces for the two ends of the allowed accumulator interval; both
 * pass through the same rounding as the kernel's result.  C_before holds C (or D before the call,
 * when accumulating).  amax_lo / amax_hi receive the interval the kernel's amax must lie in.
 * Returns the number of failing samples (first one in *first_bad). */
size_t orc_gemm_check(const orc_gemm_args *g, const void *D_got, const void *C_before,
                      const int *is, const int *js, size_t count, double err_factor,
                      float *amax_lo, float *amax_hi, int64_t *first_bad) {
  size_t bad = 0;
  float alo = 0.f, ahi = 0.f;
  unsigned char tmp[8];
  for (size_t s = 0; s < count; ++s) {
    const int i = is[s], j = js[s];
    double exact, mag;
    orc_gemm_exact(g, &i, &j, 1, &exact, &mag);
    const float cval = c_value(g, C_before, i, j);
    const float got = orc_load(g->ddt, D_got, (size_t)j * g->ldd + i, 1.f);
    int ok;
    if (!isfinite(exact) || !isfinite(mag)) {
      const float v = orc_epilogue(g, i, j, (float)exact, cval);
      orc_store(g->ddt, tmp, 0, v, g->qscale);
      const float want = orc_load(g->ddt, tmp, 0, 1.f);
      ok = same_nan_or_equal(got, want);
      if (v == v) {
        alo = fmaxf(alo, fabsf(v));
        ahi = fmaxf(ahi, fabsf(v));
      }
    } else {
      const double e = err_factor * g->k * ldexp(mag, -24) + (g->k + 1) * ldexp(mag, -52);
      const float vl = orc_epilogue(g, i, j, round_down(exact - e), cval);
      const float vh = orc_epilogue(g, i, j, round_up(exact + e), cval);
      const float vmin = fminf(vl, vh), vmax = fmaxf(vl, vh);
      float lo_out, hi_out;
      orc_store(g->ddt, tmp, 0, vmin, g->qscale);
      lo_out = orc_load(g->ddt, tmp, 0, 1.f);
      orc_store(g->ddt, tmp, 0, vmax, g->qscale);
      hi_out = orc_load(g->ddt, tmp, 0, 1.f);
      if (g->qscale < 0.f && is_fp8(g->ddt)) {
        const float t = lo_out;
        lo_out = hi_out;
        hi_out = t;
      }
      ok = got >= lo_out && got <= hi_out;
      const float mn = (vmin <= 0.f && vmax >= 0.f) ? 0.f : fminf(fabsf(vmin), fabsf(vmax));
      alo = fmaxf(alo, mn);
      ahi = fmaxf(ahi, fmaxf(fabsf(vmin), fabsf(vmax)));
    }
    if (!ok) {
      if (!bad && first_bad) *first_bad = (int64_t)s;
      ++bad;
    }
  }
  if (amax_lo) *amax_lo = alo;
  if (amax_hi) *amax_hi = ahi;
  return bad;
}

/* ---------------------------------------------------------------------------------------------
 * e5ma_adam: host scalars (src/adamw_e5m2effma.cu:150-157), per-element order
 * (src/adamw_e5m2effma.cu:17-25; include/e5m2effma.h:88-94; tests/test_adamw.cu:29-45), FP8 copy
 * and amax of |p| (src/adamw_e5m2effma.cu:70-95).  Elements [i0, i1); returns the updated amax.
 * ------------------------------------------------------------------------------------------- */
float orc_adam(const orc_adam_config *cfg, size_t count, int pdt, void *p, int gdt, const void *g,
               int mdt, void *m, void *v, int qdt, uint8_t *q, float qscale, float amax_in,
               size_t i0, size_t i1) {
  const float omb1 = (float)(1.0 - (double)cfg->beta1);
  const float omb2 = (float)(1.0 - (double)cfg->beta2);
  const float rbc1 = cfg->bias_correction ? (float)(1.0 / (1.0 - pow((double)cfg->beta1, cfg->step))) : 1.f;
  const float rbc2 = cfg->bias_correction ? (float)(1.0 / (1.0 - pow((double)cfg->beta2, cfg->step))) : 1.f;
  const float lr_wd = (float)((double)cfg->lr * cfg->weight_decay);
  const float gs = cfg->grad_scale == 0.f ? 1.f : cfg->grad_scale;
  if (i1 > count) i1 = count;
  float mx = 0.f;
  for (size_t i = i0; i < i1; ++i) {
    float gg = orc_load(gdt, g, i, 1.f) * gs;
    float pp = orc_load(pdt, p, i, 1.f);
    float mm = orc_load(mdt, m, i, 1.f), vv = orc_load(mdt, v, i, 1.f);
    if (!cfg->adamw) gg = fmaf(cfg->weight_decay, pp, gg);
    mm = fmaf(cfg->beta1, mm, omb1 * gg);
    vv = fmaf(cfg->beta2, vv, omb2 * (gg * gg));
    const float u = (mm * rbc1) / (sqrtf(vv * rbc2) + cfg->eps);
    if (cfg->adamw) pp = fmaf(-lr_wd, pp, pp);
    pp = fmaf(-cfg->lr, u, pp);
    orc_store(pdt, p, i, pp, 1.f);
    orc_store(mdt, m, i, mm, 1.f);
    orc_store(mdt, v, i, vv, 1.f);
    if (q) q[i] = qdt == ORC_E5M2 ? orc_f32_to_e5m2(pp * qscale) : orc_f32_to_e4m3(pp * qscale);
    mx = amax_fold(mx, pp);
  }
  return q ? amax_merge(amax_in, mx) : amax_in;
}

/* ---------------------------------------------------------------------------------------------
 * Quantize with the data's own amax (binds/python/e5m2effma/tensor.py:52-74, Float8Tensor.from_float)
 *
 * The reference composes this from torch operations and e5ma_cast:
 *   per tensor (:71-74): amax = x.abs().amax().clamp_min(1e-12); scale = qmax / amax;
 *                        data = e5ma_cast(x, scale=scale) (RNE satfinite of x * scale); scale_inv = 1 / scale
 *   per row    (:64-69): amax = x.abs().amax(dim=1).clamp_min(1e-12); scale = qmax / amax;
 *                        data = (x * scale[:, None]).clamp(-top, top).to(fp8); scale_inv = 1 / scale
 * with qmax = margin * top (a Python float, rounded to FP32 when it meets the FP32 tensor).  torch
 * evaluates `scalar / tensor` as tensor.reciprocal() * scalar, so scale = fl(fl(1 / amax) * qmax), and
 * torch's amax and clamp_min propagate NaN.  Clamping to +-top and then rounding gives the codes of
 * the satfinite encoder for every non-NaN value; a NaN becomes the encoder's 0x7F.
 * ------------------------------------------------------------------------------------------- */
static inline uint32_t abs_bits_max(uint32_t m, float v) {
  const uint32_t a = f2u(v) & 0x7FFFFFFFu; /* NaN patterns order above Inf: the maximum keeps a NaN */
  return a > m ? a : m;
}
static inline float quant_scale(uint32_t abits, float qmax) {
  const float a = abits > 0x7F800000u ? NAN : fmaxf(u2f(abits), 1e-12f);
  const float r = 1.0f / a;
  return r * qmax;
}

void orc_quantize(int tin, int tout, const void *src, void *dst, size_t rows, size_t cols, float sinv,
                  float qmax, int per_row, float *scale_inv, float *amax) {
  const size_t n = per_row ? cols : rows * cols, groups = per_row ? rows : 1;
  for (size_t g = 0; g < groups; ++g) {
    const size_t base = g * n;
    uint32_t ab = 0;
    for (size_t i = 0; i < n; ++i) ab = abs_bits_max(ab, orc_load(tin, src, base + i, sinv));
    const float s = quant_scale(ab, qmax);
    for (size_t i = 0; i < n; ++i) orc_store(tout, dst, base + i, orc_load(tin, src, base + i, sinv), s);
    scale_inv[g] = 1.0f / s;
    if (amax) amax[g] = u2f(ab);
  }
}
