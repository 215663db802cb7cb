// tune.cpp -- times the launch-choice candidates of struct Tuning (e5m2effma_amd/csrc/e5ma_host.hpp) on
// device 0 and records the winners for its (architecture, CU count) in e5ma_tuned.h, keeping the other
// devices' entries (the reference's tune/tune.cu:18-166 does the same for its GEMM / GEMV tables).
// Like the reference's tuner it calls the kernel launchers directly (exported by libe5m2effma.so)
// with a candidate Tuning, not through the C ABI.  A candidate replaces the default only if it is at
// least 2% faster; each time is the best of 7 runs of a batch of calls (hipEvent timing).  The cast and
// quantize candidates' outputs (codes, scale_inv, amax) are compared bit for bit with the first
// candidate's on varied inputs; one that differs is reported and never picked.
//
//   e5ma_tune [header] [--dry-run]       tune, print the entry, and (unless --dry-run) rewrite header
//   e5ma_tune --emit header arch cus splitk_div cast_grid adam_grid_bf16 adam_grid_fp32 quant_grid tail_half gemv_rows
//                [name]
//                                        rewrite header with that entry, no device use (tests)
//   e5ma_tune --ceiling                  AdamW over 2^28 parameters beside a kernel with the same memory
//                                        accesses and no arithmetic (the access pattern's own ceiling)
//
// Workloads (the BASELINE shapes of each choice):
//   cast_grid       FP32 -> E5M2 cast of 8192^2 elements, two sources rotated past the Infinity Cache
//   quant_grid      the amax pass of a per-tensor FP32 -> E5M2 quantize of 8192^2 elements (timed as the whole
//                   call, its cast pass at the cast_grid just chosen), same sources
//   adam_grid_*     AdamW over 2^28 parameters, BF16 resp. FP32 state, with an E5M2 copy
//   splitk_div      E5M2 x E5M2 -> BF16 TN GEMMs with at most 64 tiles: 512^2, 1024^2, 2048^2, 4096 x 1024
//                   and 8192 x 64, all with k = 8192 (summed), given a full workspace (e5ma_gemm_ex)
//   tail_half       0 / 1: TE wgrad (N, T) 14336 x 4096 x 8192 into FP32 with beta = 1 (896 tiles: a half-full
//                   last round) and a half-filled grid, E5M2 x E4M3 -> BF16 TN 4096 x 2048 x 8192 (summed);
//                   the candidates' outputs are compared bit for bit (half tiles must not change results)
//   gemv_rows       1 / 2 / 4 rows per wave of the n = 1 GEMV with a BF16 x: 8192 x 8192 E5M2 weights with row
//                   scales, 6 buffers rotated; outputs compared bit for bit (every choice sums a row in the same
//                   order).  The n >= 2 GEMV shapes change the summation order, so they stay compile-time choices
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <fstream>
#include <string>
#include <vector>

#include "e5ma_host.hpp"

using namespace e5ma;

static void check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    exit(1);
  }
}

template <class F> static float best_ms(F f, int batch, int reps = 7) {
  hipEvent_t a, b;
  check(hipEventCreate(&a), "hipEventCreate");
  check(hipEventCreate(&b), "hipEventCreate");
  for (int i = 0; i < batch; ++i) check(f(i), "warm-up launch");
  check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  float best = 1e30f;
  for (int r = 0; r < reps; ++r) {
    check(hipEventRecord(a, nullptr), "hipEventRecord");
    for (int i = 0; i < batch; ++i) check(f(i), "launch");
    check(hipEventRecord(b, nullptr), "hipEventRecord");
    check(hipEventSynchronize(b), "hipEventSynchronize");
    float ms = 0;
    check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
    if (ms / batch < best) best = ms / batch;
  }
  check(hipEventDestroy(a), "hipEventDestroy");
  check(hipEventDestroy(b), "hipEventDestroy");
  return best;
}

// the candidate with the best time, unless it beats the default's time by less than 2%; a candidate
// whose output differed from the first candidate's (ok[i] false) is never picked
static int pick(const char *what, const std::vector<int> &cands, const std::vector<float> &ms, int def,
                const std::vector<bool> &ok = {}) {
  const float kMargin = 0.98f;
  size_t bi = 0, di = 0;
  for (size_t i = 0; i < cands.size(); ++i) {
    const bool good = ok.empty() || ok[i];
    printf("  %-16s %8d  %9.4f ms%s\n", what, cands[i], ms[i], good ? "" : "  (output differs: rejected)");
    if (cands[i] == def) di = i;
  }
  for (size_t i = 0; i < cands.size(); ++i)
    if ((ok.empty() || ok[i]) && (ms[i] < ms[bi] || !(ok.empty() || ok[bi]))) bi = i;
  const int best = ms[bi] <= kMargin * ms[di] ? cands[bi] : def;
  printf("  -> %s = %d\n", what, best);
  return best;
}

static void *dalloc(size_t bytes, int fill) {
  void *p = nullptr;
  check(hipMalloc(&p, bytes), "hipMalloc");
  check(hipMemset(p, fill, bytes), "hipMemset");
  return p;
}

// the bytes of a device buffer
static std::vector<uint8_t> fetch(const void *p, size_t bytes) {
  std::vector<uint8_t> h(bytes);
  check(hipMemcpy(h.data(), p, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  return h;
}

// finite FP8 codes of moderate magnitude (exponent fields 12..19 for E5M2, 4..9 for E4M3), from a hash of i
__global__ void fill_codes_kernel(uint8_t *p, size_t n, uint32_t seed, int fmt) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t x = (uint32_t)i * 2654435761u ^ seed;
    x ^= x >> 13;
    x *= 0x5bd1e995u;
    x ^= x >> 15;
    p[i] = fmt == E5MA_E5M2 ? (uint8_t)((x & 0x83) | (((x >> 8) % 8 + 12) << 2))
                            : (uint8_t)((x & 0x87) | (((x >> 8) % 6 + 4) << 3));
  }
}
static void fill_codes(uint8_t *p, size_t n, uint32_t seed, int fmt) {
  fill_codes_kernel<<<4096, 256>>>(p, n, seed, fmt);
  check(hipGetLastError(), "fill_codes_kernel");
}

// AdamW's memory accesses without its arithmetic: per thread and step 8 elements of g, p, m and v read
// and p, m, v written back (16-byte accesses, non-temporal when NT, as adam.hip issues them for that
// state width) plus 8 FP8 bytes, over the same grid-stride loop.  What is stored depends on what was
// loaded (a xor), so no access is dropped.
template <int ES, bool NT>
__global__ __launch_bounds__(256) void stream_kernel(size_t count, uint8_t *p, const uint8_t *g, uint8_t *m,
                                                     uint8_t *v, uint8_t *q) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kQ = 8 * ES / 16;  // 16-byte accesses per stream and step
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
  for (size_t c = tid; c < count / 8; c += stride) {
    u32x4 G[kQ], P[kQ], M[kQ], V[kQ];
#pragma unroll
    for (int k = 0; k < kQ; ++k) {
      const size_t o = c * kQ + k;
      G[k] = NT ? __builtin_nontemporal_load((const u32x4 *)g + o) : ((const u32x4 *)g)[o];
      P[k] = NT ? __builtin_nontemporal_load((const u32x4 *)p + o) : ((const u32x4 *)p)[o];
      M[k] = NT ? __builtin_nontemporal_load((const u32x4 *)m + o) : ((const u32x4 *)m)[o];
      V[k] = NT ? __builtin_nontemporal_load((const u32x4 *)v + o) : ((const u32x4 *)v)[o];
    }
    uint32_t h = 0;
#pragma unroll
    for (int k = 0; k < kQ; ++k) {
      const size_t o = c * kQ + k;
      const u32x4 pn = P[k] ^ G[k], mn = M[k] ^ G[k], vn = V[k] ^ G[k];
      h ^= pn[0] ^ pn[1] ^ pn[2] ^ pn[3];
      if constexpr (NT) {
        __builtin_nontemporal_store(pn, (u32x4 *)p + o);
        __builtin_nontemporal_store(mn, (u32x4 *)m + o);
        __builtin_nontemporal_store(vn, (u32x4 *)v + o);
      } else {
        ((u32x4 *)p)[o] = pn;
        ((u32x4 *)m)[o] = mn;
        ((u32x4 *)v)[o] = vn;
      }
    }
    *(uint2 *)(q + 8 * c) = make_uint2(h, h >> 8);
  }
}

// AdamW (the library's kernel, the device's tuned grid) and stream_kernel on 2^28 parameters per state
// width; rates in algorithmic bytes: n * (4 reads + 3 writes of the state width + 1 FP8 byte)
static int ceiling(const DeviceInfo &di) {
  const size_t n = (size_t)1 << 28;
  for (int pt : {E5MA_BF16, E5MA_FP32}) {
    const size_t es = pt == E5MA_BF16 ? 2 : 4, bytes = n * (7 * es + 1);
    void *p = dalloc(n * es, 0x3C), *g = dalloc(n * es, 0x3A), *m = dalloc(n * es, 0x38), *v = dalloc(n * es, 0x30);
    uint8_t *q = (uint8_t *)dalloc(n, 0);
    AdamCoefficients a{};
    a.lr = 1e-4f; a.b1 = 0.9f; a.b2 = 0.999f; a.c1 = 0.1f; a.c2 = 0.001f; a.corr1 = 1.f; a.corr2 = 1.f;
    a.eps = 1e-8f; a.decay = 1e-6f; a.l2 = 0.01f; a.grad_mul = 1.f; a.decoupled = 1;
    const int grid = pt == E5MA_BF16 ? di.tune.adam_grid_bf16 : di.tune.adam_grid_fp32;
    const float adam = best_ms([&](int) {
      return launch_adam(a, n, pt, p, pt, g, pt, m, v, E5MA_E5M2, q, nullptr, nullptr, di.tune, nullptr);
    }, 3);
    const float stream = best_ms([&](int) {
      if (pt == E5MA_BF16)
        stream_kernel<2, true><<<grid, 256>>>(n, (uint8_t *)p, (const uint8_t *)g, (uint8_t *)m, (uint8_t *)v, q);
      else
        stream_kernel<4, false><<<grid, 256>>>(n, (uint8_t *)p, (const uint8_t *)g, (uint8_t *)m, (uint8_t *)v, q);
      return hipGetLastError();
    }, 3);
    printf("%s state, 2^28 parameters, grid %d: adam_kernel %.4f ms = %.1f GB/s; stream_kernel (same accesses, "
           "no arithmetic) %.4f ms = %.1f GB/s; adam / stream = %.3f\n",
           pt == E5MA_BF16 ? "BF16" : "FP32", grid, adam, bytes / (adam * 1e-3) / 1e9, stream,
           bytes / (stream * 1e-3) / 1e9, stream / adam);
    for (void *b : {p, g, m, v, (void *)q}) check(hipFree(b), "hipFree");
  }
  return 0;
}

static Tuning tune_device(const DeviceInfo &di) {
  Tuning t = di.tune, def;
  int checked = 0, differing = 0;
  // ---- cast and quantize (their outputs are compared with the first candidate's, bit for bit) ----
  {
    const size_t n = (size_t)8192 * 8192;
    void *src[2] = {dalloc(n * 4, 0x3C), dalloc(n * 4, 0x3D)};
    {  // varied values in src[0]: a sum of uniforms (roughly normal) over 12 decades, every 997th negated
      std::vector<float> h(n);
      uint32_t r = 0xE5A00Fu;
      for (size_t i = 0; i < n; ++i) {
        float v = 0.f;
        for (int q = 0; q < 4; ++q) { r ^= r << 13; r ^= r >> 17; r ^= r << 5; v += (float)(r >> 8) * 0x1p-24f - 0.5f; }
        h[i] = v * ldexpf(1.f, (int)(i % 40) - 20) * (i % 997 ? 1.f : -1.f);
      }
      check(hipMemcpy(src[0], h.data(), n * 4, hipMemcpyHostToDevice), "hipMemcpy");
    }
    void *dst = dalloc(n, 0);
    float *qs = (float *)dalloc(4, 0);
    const std::vector<int> cands = {2048, 4096, 8192, 16384, 32768};
    std::vector<float> ms;
    std::vector<bool> ok;
    std::vector<uint8_t> ref;
    float *amax = (float *)dalloc(4, 0);
    const float qscale = 1024.f;
    float *qsc = (float *)dalloc(4, 0);
    check(hipMemcpy(qsc, &qscale, 4, hipMemcpyHostToDevice), "hipMemcpy");
    for (int c : cands) {
      Tuning x = def;
      x.cast_grid = c;
      ms.push_back(best_ms([&](int i) { return launch_cast(E5MA_FP32, E5MA_E5M2, src[i & 1], dst, n, nullptr, nullptr, nullptr, x, nullptr); }, 10));
      check(hipMemset(amax, 0, 4), "hipMemset");
      check(launch_cast(E5MA_FP32, E5MA_E5M2, src[0], dst, n, nullptr, qsc, amax, x, nullptr), "launch");
      std::vector<uint8_t> out = fetch(dst, n), am = fetch(amax, 4);
      out.insert(out.end(), am.begin(), am.end());
      if (ref.empty()) ref = out;
      ok.push_back(out == ref);
      ++checked;
      differing += out != ref;
    }
    printf("cast FP32 -> E5M2, 8192^2\n");
    t.cast_grid = pick("cast_grid", cands, ms, def.cast_grid, ok);
    const std::vector<int> qc = {512, 1024, 2048, 4096, 8192, 16384};
    std::vector<float> qms;
    ok.clear();
    ref.clear();
    for (int c : qc) {
      Tuning x = def;
      x.cast_grid = t.cast_grid;
      x.quant_grid = c;
      qms.push_back(best_ms([&](int i) { return launch_quantize(E5MA_FP32, E5MA_E5M2, src[i & 1], dst, 1, n, nullptr, 57344.f, false, qs, nullptr, x, nullptr); }, 10));
      check(launch_quantize(E5MA_FP32, E5MA_E5M2, src[0], dst, 1, n, nullptr, 57344.f, false, qs, amax, x, nullptr), "launch");
      std::vector<uint8_t> out = fetch(dst, n), sc = fetch(qs, 4), am = fetch(amax, 4);
      out.insert(out.end(), sc.begin(), sc.end());
      out.insert(out.end(), am.begin(), am.end());
      if (ref.empty()) ref = out;
      ok.push_back(out == ref);
      ++checked;
      differing += out != ref;
    }
    printf("quantize FP32 -> E5M2 per tensor, 8192^2\n");
    t.quant_grid = pick("quant_grid", qc, qms, def.quant_grid, ok);
    check(hipFree(amax), "hipFree");
    check(hipFree(qsc), "hipFree");
    check(hipFree(src[0]), "hipFree");
    check(hipFree(src[1]), "hipFree");
    check(hipFree(dst), "hipFree");
    check(hipFree(qs), "hipFree");
  }
  // ---- AdamW, 2^28 parameters ----
  for (int pt : {E5MA_BF16, E5MA_FP32}) {
    const size_t n = (size_t)1 << 28, es = pt == E5MA_BF16 ? 2 : 4;
    void *p = dalloc(n * es, 0x3C), *g = dalloc(n * es, 0x3A), *m = dalloc(n * es, 0x38), *v = dalloc(n * es, 0x30);
    uint8_t *q = (uint8_t *)dalloc(n, 0);
    AdamCoefficients a{};
    a.lr = 1e-4f; a.b1 = 0.9f; a.b2 = 0.999f; a.c1 = 0.1f; a.c2 = 0.001f; a.corr1 = 1.f; a.corr2 = 1.f;
    a.eps = 1e-8f; a.decay = 1e-6f; a.l2 = 0.01f; a.grad_mul = 1.f; a.decoupled = 1;
    const std::vector<int> cands = pt == E5MA_BF16 ? std::vector<int>{16384, 32768, 65536, 131072}
                                                   : std::vector<int>{4096, 8192, 16384, 32768};
    std::vector<float> ms;
    for (int c : cands) {
      Tuning x = def;
      (pt == E5MA_BF16 ? x.adam_grid_bf16 : x.adam_grid_fp32) = c;
      ms.push_back(best_ms([&](int) { return launch_adam(a, n, pt, p, pt, g, pt, m, v, E5MA_E5M2, q, nullptr, nullptr, x, nullptr); }, 3));
    }
    printf("AdamW 2^28 parameters, %s state\n", pt == E5MA_BF16 ? "BF16" : "FP32");
    if (pt == E5MA_BF16) t.adam_grid_bf16 = pick("adam_grid_bf16", cands, ms, def.adam_grid_bf16);
    else t.adam_grid_fp32 = pick("adam_grid_fp32", cands, ms, def.adam_grid_fp32);
    for (void *b : {p, g, m, v, (void *)q}) check(hipFree(b), "hipFree");
  }
  // ---- split-K threshold ----
  {
    struct Shape { int m, n, k; };
    const Shape shapes[] = {{512, 512, 8192}, {1024, 1024, 8192}, {2048, 2048, 8192}, {4096, 1024, 8192}, {8192, 64, 8192}};
    const size_t big = (size_t)8192 * 8192;
    uint8_t *A = (uint8_t *)dalloc(big, 0x33), *B = (uint8_t *)dalloc(big, 0x35);
    void *D = dalloc(big * 2, 0);
    const Workspace ws{dalloc(kMaxWorkspace, 0), kMaxWorkspace};  // as e5ma_gemm_ex is given
    const std::vector<int> cands = {0, 2, 4, 8};
    std::vector<float> ms;
    for (int c : cands) {
      DeviceInfo x = di;
      x.tune = def;
      x.tune.splitk_div = c;
      float sum = 0;
      for (const Shape &s : shapes) {
        dev::Epilogue e{};
        e.alpha = 1.f;
        e.d = D;
        e.ldd = s.m;
        e.d_dtype = E5MA_BF16;
        e.c_dtype = E5MA_FP32;
        e.bias_dtype = E5MA_FP32;
        sum += best_ms([&](int) { return launch_gemm(E5MA_E5M2, E5MA_E5M2, true, true, A, s.k, B, s.k, s.m, s.n, s.k, e, x, ws, nullptr); }, 5);
      }
      ms.push_back(sum);
    }
    printf("GEMM TN E5M2 x E5M2 -> BF16, k = 8192, m x n in {512^2, 1024^2, 2048^2, 4096 x 1024, 8192 x 64} (summed)\n");
    t.splitk_div = pick("splitk_div", cands, ms, def.splitk_div);
    for (void *b : {(void *)A, (void *)B, D, ws.ptr}) check(hipFree(b), "hipFree");
  }
  // ---- half tiles for a half-full last round (results must not change) ----
  {
    struct Shape { int at, bt; bool akc, bkc; int m, n, k; int dt; float beta; };
    const Shape shapes[] = {{E5MA_E5M2, E5MA_E4M3, false, false, 14336, 4096, 8192, E5MA_FP32, 1.f},
                            {E5MA_E5M2, E5MA_E4M3, true, true, 4096, 2048, 8192, E5MA_BF16, 0.f}};
    const size_t big = (size_t)14336 * 8192;
    uint8_t *A = (uint8_t *)dalloc(big, 0), *B = (uint8_t *)dalloc(big, 0);
    fill_codes(A, big, 11, E5MA_E5M2);
    fill_codes(B, big, 12, E5MA_E4M3);
    void *D = dalloc((size_t)14336 * 4096 * 4, 0);
    const std::vector<int> cands = {0, 1};
    std::vector<float> ms(cands.size(), 0.f);
    std::vector<bool> ok(cands.size(), true);
    for (const Shape &sh : shapes) {
      std::vector<uint8_t> first;
      for (size_t c = 0; c < cands.size(); ++c) {
        DeviceInfo x = di;
        x.tune = def;
        x.tune.tail_half = cands[c];
        dev::Epilogue e{};
        e.alpha = 1.f;
        e.beta = sh.beta;
        e.c = sh.beta != 0.f ? D : nullptr;
        e.ldc = sh.beta != 0.f ? sh.m : 0;
        e.c_dtype = sh.dt;
        e.d = D;
        e.ldd = sh.m;
        e.d_dtype = sh.dt;
        e.bias_dtype = E5MA_FP32;
        const long long lda = sh.akc ? sh.k : sh.m, ldb = sh.bkc ? sh.k : sh.n;
        auto run = [&](int) {
          return launch_gemm(sh.at, sh.bt, sh.akc, sh.bkc, A, lda, B, ldb, sh.m, sh.n, sh.k, e, x, Workspace{}, nullptr);
        };
        // one call from a zeroed D, compared bit for bit with the first candidate's
        const size_t dbytes = (size_t)sh.m * sh.n * elem_bytes(sh.dt);
        check(hipMemset(D, 0, dbytes), "hipMemset");
        check(run(0), "launch");
        check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        std::vector<uint8_t> got = fetch(D, dbytes);
        if (c == 0) first = got;
        else if (got != first) ok[c] = false;
        ms[c] += best_ms(run, 5);
      }
    }
    printf("FP8 GEMM half tiles for a half-full last round: TE wgrad 14336 x 4096 x 8192 (N, T, FP32, beta = 1) + "
           "4096 x 2048 x 8192 TN (summed)\n");
    t.tail_half = pick("tail_half", cands, ms, def.tail_half, ok);
    for (size_t c = 1; c < cands.size(); ++c) {
      ++checked;
      if (!ok[c]) ++differing;
    }
    for (void *b : {(void *)A, (void *)B, D}) check(hipFree(b), "hipFree");
  }
  // ---- GEMV n = 1 rows per wave (results must not change) ----
  {
    const int M = 8192, K = 8192, nbuf = 6;  // 6 x 64 MiB of weights, rotated past the Infinity Cache
    std::vector<uint8_t *> W;
    for (int b = 0; b < nbuf; ++b) {
      W.push_back((uint8_t *)dalloc((size_t)M * K, 0));
      fill_codes(W.back(), (size_t)M * K, 20 + b, E5MA_E5M2);
    }
    std::vector<uint16_t> xh(K);
    for (int i = 0; i < K; ++i) xh[i] = (uint16_t)(0x3C00 + (i * 37 % 512) + (i % 3 == 0 ? 0x8000 : 0));  // BF16 x
    void *x = dalloc((size_t)K * 2, 0), *y = dalloc((size_t)M * 2, 0);
    check(hipMemcpy(x, xh.data(), xh.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    std::vector<float> sah(M);
    for (int i = 0; i < M; ++i) sah[i] = ldexpf(1.f, -6 - i % 5);
    float *sa = (float *)dalloc((size_t)M * 4, 0);
    check(hipMemcpy(sa, sah.data(), sah.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    const std::vector<int> cands = {2, 1, 4};  // the default first: the others are compared with it
    std::vector<float> ms;
    std::vector<bool> ok(cands.size(), true);
    std::vector<uint8_t> first;
    for (size_t c = 0; c < cands.size(); ++c) {
      DeviceInfo x1 = di;
      x1.tune = def;
      x1.tune.gemv_rows = cands[c];
      dev::Epilogue e{};
      e.alpha = 1.f;
      e.sa = sa;
      e.sa_vec = 1;
      e.d = y;
      e.ldd = M;
      e.d_dtype = E5MA_BF16;
      e.c_dtype = E5MA_FP32;
      e.bias_dtype = E5MA_FP32;
      auto run = [&](int i) {
        return launch_gemv(E5MA_E5M2, E5MA_BF16, W[i % nbuf], K, (const uint8_t *)x, K, M, 1, K, e, x1, nullptr);
      };
      check(run(0), "launch");
      check(hipDeviceSynchronize(), "hipDeviceSynchronize");
      std::vector<uint8_t> got = fetch(y, (size_t)M * 2);
      if (c == 0) first = got;
      else if (got != first) ok[c] = false;
      ms.push_back(best_ms(run, 30));
    }
    printf("GEMV n = 1, 8192 x 8192 E5M2 (row scales) x BF16 -> BF16, weights rotated over 6 buffers\n");
    t.gemv_rows = pick("gemv_rows", cands, ms, def.gemv_rows, ok);
    for (size_t c = 1; c < cands.size(); ++c) {
      ++checked;
      if (!ok[c]) ++differing;
    }
    for (uint8_t *b : W) check(hipFree(b), "hipFree");
    for (void *b : {x, y, (void *)sa}) check(hipFree(b), "hipFree");
  }
  printf("outputs of %d cast / quantize / half-tile / GEMV candidates compared with their first candidate's: %d differ\n",
         checked, differing);
  return t;
}

// rewrite the header: every entry line of other devices, then this device's
static int emit(const char *path, const char *arch, int cus, const Tuning &t, const char *name) {
  std::vector<std::string> keep;
  {
    std::ifstream in(path);
    std::string line;
    char ea[64];
    int ec = 0;
    while (std::getline(in, line)) {
      const size_t pos = line.find("/* entry arch=");
      if (pos == std::string::npos) continue;
      if (sscanf(line.c_str() + pos, "/* entry arch=%63s cus=%d", ea, &ec) == 2 && !(strcmp(ea, arch) == 0 && ec == cus))
        keep.push_back(line);
    }
  }
  char buf[512];
  snprintf(buf, sizeof buf, "  {\"%s\", %d, {%d, %d, %d, %d, %d, %d, %d}}, /* entry arch=%s cus=%d tuned on %s */ \\",
           arch, cus, t.splitk_div, t.cast_grid, t.adam_grid_bf16, t.adam_grid_fp32, t.quant_grid, t.tail_half, t.gemv_rows,
           arch, cus, name);
  keep.push_back(buf);
  std::ofstream out(path);
  if (!out) {
    fprintf(stderr, "cannot write %s\n", path);
    return 1;
  }
  out << "// e5ma_tuned.h -- written by the tuner (e5m2effma_amd/tune/tune.cpp; make -C e5m2effma_amd/csrc tune-run):\n"
         "// per-device launch choices of struct Tuning (e5ma_host.hpp), one entry per (architecture, CU count):\n"
         "// {arch, cus, {splitk_div, cast_grid, adam_grid_bf16, adam_grid_fp32, quant_grid, tail_half, gemv_rows}}.\n"
         "// Re-running the tuner on a device adds or replaces that device's entry and keeps the others.\n"
         "#pragma once\n#define E5MA_TUNED_ENTRIES \\\n";
  for (const std::string &l : keep) out << l << "\n";
  out << "\n";
  printf("wrote %s: %s\n", path, buf);
  return 0;
}

int main(int argc, char **argv) {
  if (argc >= 12 && strcmp(argv[1], "--emit") == 0) {
    Tuning t;
    t.splitk_div = atoi(argv[5]);
    t.cast_grid = atoi(argv[6]);
    t.adam_grid_bf16 = atoi(argv[7]);
    t.adam_grid_fp32 = atoi(argv[8]);
    t.quant_grid = atoi(argv[9]);
    t.tail_half = atoi(argv[10]);
    t.gemv_rows = atoi(argv[11]);
    return emit(argv[2], argv[3], atoi(argv[4]), t, argc > 12 ? argv[12] : "unnamed device");
  }
  const char *path = "e5m2effma_amd/csrc/e5ma_tuned.h";
  bool dry = false, ceil_only = false;
  for (int i = 1; i < argc; ++i) {
    if (strcmp(argv[i], "--dry-run") == 0) dry = true;
    else if (strcmp(argv[i], "--ceiling") == 0) ceil_only = true;
    else path = argv[i];
  }
  check(hipSetDevice(0), "hipSetDevice");
  {
    Call call;
    int dev = 0;
    if (e5ma_status st = resolve_device(call, &dev)) {
      fprintf(stderr, "device 0 is not supported (status %d): %s\n", (int)st, thread_message());
      return 1;
    }
  }
  const DeviceInfo &di = device_info(0);
  hipDeviceProp_t p;
  check(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
  char arch[64];
  snprintf(arch, sizeof arch, "%s", p.gcnArchName);
  if (char *c = strchr(arch, ':')) *c = 0;
  char name[256];
  snprintf(name, sizeof name, "%s", p.name[0] ? p.name : "an unnamed device");  // empty without amdgpu.ids
  if (ceil_only) {
    printf("AdamW access-pattern ceiling on %s (%s, %d CUs)\n", name, arch, di.cus);
    return ceiling(di);
  }
  printf("tuning on %s (%s, %d CUs)\n", name, arch, di.cus);
  const Tuning t = tune_device(di);
  printf("entry: {\"%s\", %d, {%d, %d, %d, %d, %d, %d, %d}}\n", arch, di.cus, t.splitk_div, t.cast_grid,
         t.adam_grid_bf16, t.adam_grid_fp32, t.quant_grid, t.tail_half, t.gemv_rows);
  return dry ? 0 : emit(path, arch, di.cus, t, name);
}
