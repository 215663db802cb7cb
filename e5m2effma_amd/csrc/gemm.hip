// gemm.hip -- kernel choice for the tiled path of e5ma_gemm (reference src/gemm_e5m2effma.cu:18-39), and
// split-K for outputs with fewer 256 x 256 tiles than the device has compute units.
//
// Split-K: the fast kernel runs with grid = tiles x S, block (tile, s) reducing the s-th of S equal K
// ranges into FP32 partials (a workspace of S * ldw * n floats, ldw = m rounded up to 4, allocated and
// freed in stream order from the library's memory pool of the device, which keeps it mapped);
// splitk_reduce_kernel then adds the S partials of every output in split order (deterministic) and
// applies the epilogue (alpha * sa * sb, bias, beta * C, conversion, amax).  Each split's error terms are
// the unsplit kernel's over a part of the products, so the accumulation bound of the whole K still holds,
// with S - 1 FP32 additions on top (S <= 256: far inside 2 k 2^-24 sum|a b|).  Splitting is used only
// when the tiles fill at most 1 / Tuning::splitk_div of the CUs (default 4: 2 splits of a half-filled
// grid measured slower than none, the partials' traffic outweighing the idle half); S is then the
// largest divisor of the ring rounds in K that keeps tiles * S <= CUs and at least two rounds per split.
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {
namespace {

using namespace dev;

constexpr int kTile = 256;                             // the fast kernels' block tile
constexpr long long kMaxWorkspace = 1LL << 30;         // bytes of FP32 partials, at most
constexpr int kReduceThreads = 256;

int split_count(int m, int n, int k, int round, int cus, int div) {
  const long long tiles = (long long)((m + kTile - 1) / kTile) * ((n + kTile - 1) / kTile);
  if (div <= 0 || tiles * div > cus) return 1;
  const int rounds = k / round;
  const long long ldw = (m + 3) & ~3LL;
  int best = 1;
  for (int s = 2; s <= rounds / 2 && tiles * s <= cus; ++s)
    if (rounds % s == 0 && s * ldw * n * 4 <= kMaxWorkspace) best = s;
  return best;
}

// out(i, j) = epilogue(sum_s ws[s][j][i]); thread q takes rows 4 (q % rows4) .. + 3 of column q / rows4
__global__ __launch_bounds__(kReduceThreads) void splitk_reduce_kernel(const float *ws, long long ldw, long long sstride,
                                                                      int splits, int m, int n, Epilogue e) {
  __shared__ float red[kReduceThreads / 64];
  const EpiState st = epi_begin(e);
  const long long rows4 = (m + 3) / 4, total = rows4 * n;
  float mx = 0.f;
  for (long long q = (long long)blockIdx.x * kReduceThreads + threadIdx.x; q < total;
       q += (long long)gridDim.x * kReduceThreads) {
    const int j = (int)(q / rows4), i = (int)(q - j * rows4) * 4;
    const float *p = ws + (long long)j * ldw + i;
    float4 sum = *(const float4 *)p;
    for (int s = 1; s < splits; ++s) {
      const float4 v = *(const float4 *)(p + s * sstride);
      sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
    const float a[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (i + r < m) {
        const float v = epi_value(e, st, i + r, j, a[r]);
        store_any(e.d_dtype, e.d, (size_t)j * e.ldd + i + r, v, st.qscale);
        mx = amax_fold(mx, v);
      }
  }
  if (e.amax) amax_commit_block(e.amax, mx, red);
}

typedef hipError_t (*FastLaunch)(int, int, bool, bool, const uint8_t *, long long, const uint8_t *, long long, int, int,
                                 int, int, const Epilogue &, hipStream_t);

hipError_t launch_fast(FastLaunch launch, int round, int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda,
                       const uint8_t *B, long long ldb, int m, int n, int k, const Epilogue &e, const DeviceInfo &di,
                       hipStream_t s) {
  const int splits = split_count(m, n, k, round, di.cus > 0 ? di.cus : 256, di.tune.splitk_div);
  if (splits > 1) {
    const long long ldw = (m + 3) & ~3LL;
    void *ws = nullptr;
    const size_t bytes = (size_t)splits * ldw * n * sizeof(float);
    if (di.pool && hipMallocFromPoolAsync(&ws, bytes, di.pool, s) == hipSuccess) {
      Epilogue part{};  // raw FP32 partials: alpha 1, no scales, bias, C or amax
      part.alpha = 1.f;
      part.d = ws;
      part.ldd = ldw;
      part.d_dtype = E5MA_FP32;
      hipError_t err = launch(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, splits, part, s);
      if (err == hipSuccess) {
        const long long total = (m + 3) / 4 * (long long)n;
        const int grid = (int)std::min<long long>((total + kReduceThreads - 1) / kReduceThreads, 8192);
        splitk_reduce_kernel<<<grid, kReduceThreads, 0, s>>>((const float *)ws, ldw, ldw * n, splits, m, n, e);
        err = hipGetLastError();
      }
      const hipError_t ferr = hipFreeAsync(ws, s);
      return err != hipSuccess ? err : ferr;
    }
    (void)hipGetLastError();  // no workspace: run unsplit
  }
  return launch(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, 1, e, s);
}

}  // namespace

hipError_t launch_gemm(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                       long long ldb, int m, int n, int k, const dev::Epilogue &e, const DeviceInfo &di,
                       hipStream_t s) {
  if (gemm_f8_applies(at, bt, akc, bkc, m, n, k, lda, ldb))
    return launch_fast(launch_gemm_f8, gemm_f8_round(), at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, di, s);
  if (gemm_h_applies(at, bt, akc, bkc, m, n, k))
    return launch_fast(launch_gemm_h, gemm_h_round(bt), at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, di, s);
  return launch_gemm_generic(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
}

}  // namespace e5ma
