// gemm.hip -- kernel choice for the tiled path of e5ma_gemm (reference src/gemm_e5m2effma.cu:18-39), and
// split-K for outputs with fewer 256 x 256 tiles than the device has compute units, where the caller
// supplies device memory for it (e5ma_gemm_ex, e5ma_gemm_noalloc; e5ma_gemm never splits).
//
// Split-K: the fast kernel runs with grid = tiles x S, block (tile, s) reducing the s-th of S equal K
// ranges into FP32 partials (S * ldw * n floats of the workspace, ldw = m rounded up to 4);
// splitk_reduce_kernel then adds the S partials of every output in split order (deterministic) and
// applies the epilogue (alpha * sa * sb, bias, beta * C, conversion, amax).  Each split's error terms are
// the unsplit kernel's over a part of the products, so the accumulation bound of the whole K still holds,
// with S - 1 FP32 additions on top (S <= 256: far inside 2 k 2^-24 sum|a b|); the bits may differ from
// the unsplit result's.  Splitting is used only when the tiles fill at most 1 / Tuning::splitk_div of the
// CUs (default 4: 2 splits of a half-filled grid measured slower than none, the partials' traffic
// outweighing the idle half); S is then the largest divisor of the ring rounds in K that keeps
// tiles * S <= CUs, at least two rounds per split and the partials within the workspace (at most
// kMaxWorkspace).  A smaller workspace gives fewer splits; none at all, an unsplit launch.
#include "e5ma_host.hpp"
#include "gemm_common.hpp"

namespace e5ma {
namespace {

using namespace dev;

constexpr int kTile = 256;  // the fast kernels' block tile
constexpr int kReduceThreads = 256;

long long partial_ld(int m) { return (m + 3) & ~3LL; }
size_t partial_bytes(int splits, int m, int n) { return (size_t)splits * partial_ld(m) * n * sizeof(float); }

// splits of K for this shape with at most `cap` bytes of partials (1: none)
int split_count(int m, int n, int k, int round, int cus, int div, size_t cap) {
  const long long tiles = (long long)((m + kTile - 1) / kTile) * ((n + kTile - 1) / kTile);
  if (div <= 0 || tiles * div > cus) return 1;
  const int rounds = k / round;
  int best = 1;
  for (int s = 2; s <= rounds / 2 && tiles * s <= cus; ++s)
    if (rounds % s == 0 && partial_bytes(s, m, n) <= cap) best = s;
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
                                 int, int, int, int, const Epilogue &, hipStream_t);

hipError_t launch_fast(FastLaunch launch, int round, int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda,
                       const uint8_t *B, long long ldb, int m, int n, int k, const Epilogue &e, const DeviceInfo &di,
                       const Workspace &ws, hipStream_t s) {
  const size_t cap = ws.ptr ? std::min(ws.bytes, kMaxWorkspace) : 0;
  const int splits = split_count(m, n, k, round, di.cus > 0 ? di.cus : 256, di.tune.splitk_div, cap);
  if (splits == 1) {
    return launch(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, 1, di.cus, di.tune.tail_half, e, s);
  }
  const long long ldw = partial_ld(m);
  Epilogue part{};  // raw FP32 partials: alpha 1, no scales, bias, C or amax
  part.alpha = 1.f;
  part.d = ws.ptr;
  part.ldd = ldw;
  part.d_dtype = E5MA_FP32;
  part.c_dtype = E5MA_FP32;
  part.bias_dtype = E5MA_FP32;
  hipError_t err = launch(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, splits, di.cus, 0, part, s);
  if (err != hipSuccess) return err;
  const long long total = (m + 3) / 4 * (long long)n;
  const int grid = (int)std::min<long long>((total + kReduceThreads - 1) / kReduceThreads, 8192);
  splitk_reduce_kernel<<<grid, kReduceThreads, 0, s>>>((const float *)ws.ptr, ldw, ldw * n, splits, m, n, e);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(int at, int bt, bool akc, bool bkc, const uint8_t *A, long long lda, const uint8_t *B,
                       long long ldb, int m, int n, int k, const dev::Epilogue &e, const DeviceInfo &di,
                       const Workspace &ws, hipStream_t s) {
  if (gemm_f8_applies(at, bt, akc, bkc, m, n, k, lda, ldb))
    return launch_fast(launch_gemm_f8, gemm_f8_round(), at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, di, ws, s);
  if (gemm_h_applies(at, bt, akc, bkc, m, n, k))
    return launch_fast(launch_gemm_h, gemm_h_round(bt), at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, di, ws, s);
  return launch_gemm_generic(at, bt, akc, bkc, A, lda, B, ldb, m, n, k, e, s);
}

size_t gemm_workspace_bytes(int at, int bt, bool akc, bool bkc, int m, int n, int k, long long lda, long long ldb,
                            const DeviceInfo &di) {
  int round = 0;
  if (gemm_f8_applies(at, bt, akc, bkc, m, n, k, lda, ldb)) round = gemm_f8_round();
  else if (gemm_h_applies(at, bt, akc, bkc, m, n, k)) round = gemm_h_round(bt);
  else return 0;  // the generic kernel does not split
  const int splits = split_count(m, n, k, round, di.cus > 0 ? di.cus : 256, di.tune.splitk_div, kMaxWorkspace);
  return splits > 1 ? partial_bytes(splits, m, n) : 0;
}

}  // namespace e5ma
