/* e5ma_oracle.h -- CPU restatement of the reference's FP8 compute semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this code, and only as the checker (or the timed CPU baseline); the product library
 * (e5m2effma_amd) never calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (/root/reference = srose69/e5m2effma 0.2.0).  Built with -O2 -ffp-contract=off, no fast-math,
 * so each FP32 operation below rounds exactly once, as written.
 */
#ifndef E5MA_ORACLE_H
#define E5MA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_E4M3 = 0, ORC_BF16 = 1, ORC_FP16 = 2, ORC_FP32 = 3, ORC_E5M2 = 4 };

/* ---- scalar codecs ---- */
float orc_e4m3_value(uint8_t b);
float orc_e5m2_value(uint8_t b);
float orc_e4m3_operand(uint8_t b);
float orc_e5m2_operand(uint8_t b);
float orc_bf16_value(uint16_t h);
float orc_f16_value(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
uint16_t orc_f32_to_f16(float x);
uint8_t orc_f32_to_e4m3(float x);
uint8_t orc_f32_to_e5m2(float x);
uint8_t orc_fp8_encode_search(float x, int fmt);
float orc_load(int dtype, const void *p, size_t i, float sinv);
void orc_store(int dtype, void *p, size_t i, float v, float qscale);
uint16_t orc_lane(uint8_t a, uint8_t b, uint16_t acc, int fa, int fb);

/* ---- batch helpers (numpy-friendly) ---- */
void orc_encode_batch(int dtype, const float *x, void *out, size_t n, float qscale);
void orc_decode_batch(int dtype, const void *p, float *out, size_t n, float sinv);
void orc_lane_batch(const uint8_t *a, const uint8_t *b, const uint16_t *acc, int fa, int fb,
                    uint16_t *out, size_t n);
typedef uint32_t (*orc_ref_lane_fn)(uint32_t, uint32_t, uint32_t, int, int);
size_t orc_lane_compare(orc_ref_lane_fn ref, const uint16_t *accs, size_t nacc, int fa, int fb,
                        uint32_t *first_bad);
void orc_lane_gemm(orc_ref_lane_fn fn, const uint8_t *a, const uint8_t *b, int N, int K, int fa, int fb,
                   uint16_t *out, int row0, int row1);
void orc_lane_sweep(orc_ref_lane_fn fn, const uint16_t *accs, size_t nacc, int fa, int fb,
                    uint16_t *out);
size_t orc_encode_selfcheck(int fmt, uint64_t start, uint64_t stop, uint64_t step, uint32_t *first_bad);

/* ---- cast ---- */
float orc_cast(int tin, int tout, const void *src, void *dst, size_t count, float sinv,
               float qscale, float amax_in);

/* ---- quantize with the data's own amax (Float8Tensor.from_float) ---- */
void orc_quantize(int tin, int tout, const void *src, void *dst, size_t rows, size_t cols, float sinv,
                  float qmax, int per_row, float *scale_inv, float *amax);

/* ---- GEMM ---- */
typedef struct {
  int transa, transb, m, n, k;
  float alpha;
  int adt; const void *A; int lda; const float *sa; int sa_vec;
  int bdt; const void *B; int ldb; const float *sb; int sb_vec;
  float beta;
  int cdt; const void *C; int ldc; float csinv;   /* C == NULL with beta != 0: C = D (accumulate) */
  int ddt; void *D; int ldd; float qscale;
  int biasdt; const void *bias;                  /* NULL: no bias */
  int ocp_operands;                              /* 1: FP8 Inf / NaN operand codes stay Inf / NaN */
} orc_gemm_args;

float orc_epilogue(const orc_gemm_args *g, int i, int j, float acc, float cval);
float orc_gemm_chain(const orc_gemm_args *g, float amax_in, int row0, int row1, int nthreads);
void orc_gemm_exact(const orc_gemm_args *g, const int *is, const int *js, size_t count,
                    double *exact, double *mag);
size_t orc_gemm_check(const orc_gemm_args *g, const void *D_got, const void *C_before,
                      const int *is, const int *js, size_t count, double err_factor,
                      float *amax_lo, float *amax_hi, int64_t *first_bad);

/* ---- Adam / AdamW ---- */
typedef struct {
  float lr, beta1, beta2, eps, weight_decay;
  int step, adamw, bias_correction;
  float grad_scale;
} orc_adam_config;

float orc_adam(const orc_adam_config *cfg, size_t count, int pdt, void *p, int gdt, const void *g,
               int mdt, void *m, void *v, int qdt, uint8_t *q, float qscale, float amax_in,
               size_t i0, size_t i1);

#ifdef __cplusplus
}
#endif
#endif
