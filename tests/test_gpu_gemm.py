"""Tiled e5ma_gemm on the GPU against the oracle's bound
|acc - exact| <= 2 * k * 2^-24 * sum|a*b| (exact products, FP32 accumulation in another order than the
reference's FFMA chain), with the epilogue applied to both ends of the interval (oracle
orc_gemm_check).  Mirrors the reference's coverage (tests/test_gemm.cu:13-46): 16 dtype pairs x 4
layouts, m / n tails, every output dtype, C of another dtype, accumulate, bias, outer scaling."""
import itertools

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
E5, E4, B16, F32, F16 = oracle.E5M2, oracle.E4M3, oracle.BF16, oracle.FP32, oracle.FP16
OPERANDS = [E5, E4, B16, F32]
LAYOUTS = [(1, 0), (0, 0), (0, 1), (1, 1)]


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


@pytest.mark.parametrize("adt,bdt", list(itertools.product(OPERANDS, OPERANDS)))
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_pairs_and_layouts(dev, adt, bdt, ta, tb):
    rng = np.random.default_rng(adt * 100 + bdt * 10 + ta * 2 + tb)
    case = gu.GemmCase(rng, ta, tb, 67, 45, 80, adt, bdt, ddt=F32, alpha=1.25, sa=0.37, sb=1.9, beta=0.5, cdt=F32,
                       biasdt=F32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ddt", [B16, F16, F32, E5, E4])
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 0)])
def test_output_dtypes_and_amax(dev, ddt, ta, tb):
    rng = np.random.default_rng(ddt + 10 * ta)
    qs = 0.25 if ddt in gu.FP8 else None
    case = gu.GemmCase(rng, ta, tb, 96, 80, 128, E5, E4, ddt=ddt, sa=0.5, sb=0.75, qscale=qs, amax=True)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("cdt", [B16, F16, F32, E5, E4])
def test_c_of_every_dtype(dev, cdt):
    rng = np.random.default_rng(cdt)
    case = gu.GemmCase(rng, 1, 0, 72, 40, 64, E4, E5, ddt=B16, beta=-0.75, cdt=cdt, csinv=0.5, biasdt=B16)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt,bdt", [(E5, E4), (E5, B16), (B16, F32)])
def test_accumulate_into_fp32_main_grad(dev, adt, bdt):
    """TE 'accumulate': C = NULL, beta = 1, FP32 D (reference src/gemm_e5m2effma.cu:83)."""
    rng = np.random.default_rng(3)
    case = gu.GemmCase(rng, 1, 0, 130, 70, 96, adt, bdt, ddt=F32, beta=1.0, cdt=None, biasdt=F32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_outer_scaling(dev, ta, tb):
    rng = np.random.default_rng(ta * 2 + tb + 40)
    m, n = 100, 52
    sa = (0.25 + rng.integers(0, 1024, m) / 512).astype(np.float32)  # reference tests/test_util.h:96-97
    sb = (0.25 + rng.integers(0, 1024, n) / 512).astype(np.float32)
    case = gu.GemmCase(rng, ta, tb, m, n, 64, E5, E4, ddt=B16, alpha=0.5, sa=sa, sb=sb)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("m,n,k", [(1, 9, 16), (31, 33, 16), (129, 130, 48), (255, 257, 1040), (64, 64, 0),
                                   (200, 16, 4096)])
@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E4, B16), (F32, E5)])
def test_shapes(dev, m, n, k, adt, bdt):
    rng = np.random.default_rng(m + n + k)
    case = gu.GemmCase(rng, 1, 0, m, n, k, adt, bdt, ddt=B16, sa=0.5, biasdt=F32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E5, E4), (E4, E5), (E4, E4), (E5, B16), (B16, E4)])
def test_single_product_is_exact(dev, adt, bdt):
    """k = 16 with one non-zero term per output: D (FP32) = a * b exactly for every pair of codes, so the
    matrix cores' products are exact, subnormals included (reference docs/numerics.md:3-28)."""
    m = n = 256
    k = 16

    def codes(dt):
        if dt in gu.FP8:
            c = np.arange(256, dtype=np.uint8)
            bad = (c & 0x7C) == 0x7C if dt == E5 else (c & 0x7F) == 0x7F
            c[bad] = 0
            return c
        rng = np.random.default_rng(1)
        return oracle.encode(B16, rng.standard_normal(256).astype(np.float32))
    a, b = codes(adt), codes(bdt)
    A = np.zeros(k * m, gu.NPD[adt])
    B = np.zeros(k * n, gu.NPD[bdt])
    A[np.arange(m) * k + 5] = a
    B[np.arange(n) * k + 5] = b
    case = gu.GemmCase(None, 1, 0, m, n, k, adt, bdt, ddt=F32, pad=0, A=A, B=B)
    s, D, _ = case.run(dev)
    assert s == 0
    va = oracle.decode(adt, a).astype(np.float64)
    vb = oracle.decode(bdt, b).astype(np.float64)
    want = np.outer(vb, va).astype(np.float32)  # [j][i]
    got = D.reshape(n, case.ldd)[:, :m]
    assert np.array_equal(got, want)


def test_config1_512_row_major(dev):
    """BASELINE config 1 shape through the C ABI: row-major a @ b, 512^3, E5M2 x E5M2 -> BF16, N(0,1)*4
    inputs, issued column-major as out^T = b^T a^T (e5ma_gemm(N, N, 512, 512, 512, A := b, B := a))."""
    rng = np.random.default_rng(0xE5A001)
    case = gu.GemmCase(rng, 0, 0, 512, 512, 512, E5, E5, ddt=B16, pad=0, dist="normal", sigma=4.0, sa=1.0, sb=1.0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_large_sampled(dev, ta, tb):
    rng = np.random.default_rng(77 + ta * 2 + tb)
    case = gu.GemmCase(rng, ta, tb, 1024, 768, 2048, E5, E4, ddt=B16, dist="normal", sigma=8.0, sa=1 / 64,
                       sb=1 / 64, pad=0)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=8192, rng=rng)
    assert bad == 0, first


def test_inf_nan_operands_propagate(dev):
    """FP8 operand Inf / NaN codes are outside the contract; the matrix cores read them as OCP Inf / NaN,
    so an E5M2 output saturates (Inf -> 0x7B / 0xFB), NaN -> 0x7F, and amax (NaN ignored) becomes Inf
    (BASELINE config 4 run 3 semantics)."""
    rng = np.random.default_rng(12)
    m, n, k = 64, 48, 64
    case = gu.GemmCase(rng, 1, 0, m, n, k, E4, E5, ddt=E5, qscale=1.0, amax=True, pad=0, dist="normal", sigma=0.5)
    B = case.B.copy()
    B[5 * k + 3] = 0x7C   # +Inf in column 5
    B[9 * k + 7] = 0xFC   # -Inf in column 9
    B[20 * k + 1] = 0x7E  # NaN in column 20
    case.B = B
    s, D, amax = case.run(dev)
    assert s == 0
    bad, first = case.check(D)
    assert bad == 0, first
    assert amax == np.inf


# ---- the FP8 matrix-core path (k >= 8192) ---------------------------------------------------------
def test_f8_path_worst_case_groups(dev):
    """Every group of 8 consecutive k holds one product 2^e and seven products just below 2^(e - 13),
    which the FP8 matrix cores truncate to zero (the worst case of their accumulation).  At k = 8192 the
    result must still satisfy the contract bound 2 * k * 2^-24 * sum|a*b|."""
    rng = np.random.default_rng(8192)
    m, n, k = 64, 32, 8192
    E5c = lambda v: oracle.encode(E5, np.asarray(v, np.float32))
    A = np.zeros((m, k), np.uint8)
    groups = k // 8
    e = rng.integers(0, 14, (m, groups)).astype(np.float32)  # small terms stay E5M2 normals
    sign = np.where(rng.integers(0, 2, (m, groups)) == 1, -1.0, 1.0).astype(np.float32)
    A[:, 0::8] = E5c(sign * 2.0 ** e)
    for t in range(1, 8):
        A[:, t::8] = E5c(sign * 1.75 * 2.0 ** (e - 14))
    B = np.full((n, k), E5c([1.0])[0], np.uint8)
    case = gu.GemmCase(None, 1, 0, m, n, k, E5, E5, ddt=F32, pad=0, A=A.ravel(), B=B.ravel())
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E5, E4), (E4, E5), (E4, E4)])
def test_f8_path_uniform_codes(dev, adt, bdt):
    rng = np.random.default_rng(adt * 10 + bdt + 8192)
    case = gu.GemmCase(rng, 1, 0, 160, 96, 8192, adt, bdt, ddt=F32, alpha=0.5, sa=0.37, sb=1.9, biasdt=F32,
                       beta=0.5, cdt=B16, pad=0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_f8_path_layouts(dev, ta, tb):
    rng = np.random.default_rng(ta * 2 + tb + 8193)
    case = gu.GemmCase(rng, ta, tb, 200, 136, 8192 + 16, E5, E4, ddt=E5, qscale=0.5, amax=True, sa=0.25, sb=2.0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


# ---- the fast FP8 kernel in every layout (k a multiple of 256; an M / N-contiguous operand needs
# m / n a multiple of 16): tiles of 256 x 256 with m / n tails, the transposing LDS reads of
# M / N-contiguous operands --------------------------------------------------------------------------
@pytest.mark.parametrize("adt,bdt", [(E5, E4), (E4, E5)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_f8_fast_layouts(dev, ta, tb, adt, bdt):
    rng = np.random.default_rng(ta * 4 + tb * 2 + adt + 8320)
    case = gu.GemmCase(rng, ta, tb, 272, 304, 8192, adt, bdt, ddt=B16, pad=32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_f8_fast_layouts_full_epilogue(dev, ta, tb):
    """OUTER scale vectors, alpha, bias and accumulation into D (beta = 1, C = NULL), FP32 output."""
    rng = np.random.default_rng(ta * 2 + tb + 8400)
    m, n = 288, 160
    sa = rng.uniform(0.25, 2.0, m).astype(np.float32)
    sb = rng.uniform(0.25, 2.0, n).astype(np.float32)
    case = gu.GemmCase(rng, ta, tb, m, n, 8192, E5, E5, ddt=F32, alpha=0.75, sa=sa, sb=sb, biasdt=B16, beta=1.0,
                       dist="normal", sigma=4.0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_f8_fast_layouts_fp8_output(dev, ta, tb):
    rng = np.random.default_rng(ta * 2 + tb + 8500)
    case = gu.GemmCase(rng, ta, tb, 256, 512, 8192, E4, E4, ddt=E5, qscale=0.5, amax=True, sa=0.25, sb=2.0,
                       dist="normal", sigma=2.0, pad=0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb,adt,bdt,ddt,k,m,n", [(1, 0, E5, E4, E5, 8192, 528, 304),
                                                     (0, 0, E4, E5, E4, 8192, 528, 304),
                                                     (0, 1, E5, E5, E5, 8192, 528, 304),
                                                     (1, 1, E4, E4, E4, 8192, 528, 304),
                                                     (1, 0, E4, B16, E5, 1024, 528, 304),
                                                     (0, 1, E5, E4, E4, 1024, 528, 304),
                                                     (1, 0, E5, E5, E5, 8192, 16, 16),
                                                     (1, 1, E5, E4, E4, 8192, 768, 512)])
def test_fp8_output_staged_as_codes(dev, ta, tb, adt, bdt, ddt, k, m, n):
    """FP8 D with 16-byte aligned columns (ldd % 16 == 0, m % 16 == 0), no bias, beta = 0: the write-out that
    stages the tile as FP8 codes, on both matrix-core kernels.  m = 528, n = 304 give full tiles and edge
    tiles in both directions (16 rows, 48 columns); 16 x 16 is a single edge tile; 768 x 512 full tiles only.
    Row-wise sa and column-wise sb (none for a BF16 B), scale and amax; Inf / NaN codes in A make saturated
    and NaN outputs.  The padding rows of D (ldd = m + 16) must stay untouched."""
    rng = np.random.default_rng(ta * 2 + tb + 16 * ddt + k + m)
    sa = rng.uniform(0.25, 2.0, m).astype(np.float32)
    sb = rng.uniform(0.25, 2.0, n).astype(np.float32) if bdt != B16 else None
    case = gu.GemmCase(rng, ta, tb, m, n, k, adt, bdt, ddt=ddt, alpha=0.75, sa=sa, sb=sb, qscale=4.0, amax=True,
                       pad=0, ldd=m + 16, dist="normal", sigma=2.0)
    A = case.A.copy()
    inf, nan = (0x7C, 0x7E) if adt == E5 else (0x7F, 0x7F)  # E4M3 has no Inf: NaN codes only
    for r, code in ((3, inf), (min(300, m - 2), nan), (m - 8, inf | 0x80)):  # row m - 8: the last 16-row chunk
        A[r * case.lda + 5 if ta else 5 * case.lda + r] = code
    case.A = A
    s, D, amax = case.run(dev)
    assert s == 0, s
    bad, first = case.check(D, amax)
    assert bad == 0, first
    assert np.isinf(amax) == (adt == E5), amax


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1)])
def test_f8_fast_mn_tails_fall_back(dev, ta, tb):
    """m not a multiple of 16 with an M-contiguous A: the general kernel takes the call."""
    rng = np.random.default_rng(ta * 2 + tb + 8600)
    case = gu.GemmCase(rng, ta, tb, 100, 48, 8192, E5, E4, ddt=F32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


def test_config4_dgrad_shape(dev):
    """TE dgrad: dX = W^T dY, e5ma_gemm(N, N, in, batch, out) with W E4M3 N(0, 0.02)
    (M-contiguous), dY E5M2 N(0, 1e-3), row-wise scale_inv vectors on both, BF16 out.  k = out = 14336
    as in the config; m, n reduced (sampled check)."""
    rng = np.random.default_rng(14336)
    m, n, k = 512, 384, 14336
    W = oracle.encode(E4, (rng.standard_normal(m * k) * 0.02 * 64).astype(np.float32))
    dY = oracle.encode(E5, (rng.standard_normal(k * n) * 1e-3 * 1024).astype(np.float32))
    sa = np.full(m, 1 / 64, np.float32) * rng.uniform(0.5, 2, m).astype(np.float32)
    sb = np.full(n, 1 / 1024, np.float32) * rng.uniform(0.5, 2, n).astype(np.float32)
    case = gu.GemmCase(None, 0, 0, m, n, k, E4, E5, ddt=B16, sa=sa, sb=sb, pad=0, A=W, B=dY)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


def test_config4_wgrad_shape(dev):
    """TE wgrad: main_grad += dY X^T + bias, e5ma_gemm(N, T, out, in, batch, beta = 1,
    C = NULL) with dY E5M2 (M-contiguous) and X E4M3 (N-contiguous), FP32 D.  k = batch = 8192; m, n
    reduced (sampled check)."""
    rng = np.random.default_rng(8192 + 4096)
    m, n, k = 768, 512, 8192
    dY = oracle.encode(E5, (rng.standard_normal(m * k) * 1e-3 * 1024).astype(np.float32))
    X = oracle.encode(E4, (rng.standard_normal(k * n) * 0.5).astype(np.float32))
    case = gu.GemmCase(rng, 0, 1, m, n, k, E5, E4, ddt=F32, sa=1 / 1024, sb=1.0, beta=1.0, biasdt=F32, pad=0,
                       A=dY, B=X, D0=rng.uniform(-1, 1, (m + 3) * n).astype(np.float32))
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


def test_config4_e5m2_output_inf_nan(dev):
    """Config 4 run 3: dgrad layout with E5M2 output, scale and amax, and about 0.001 % of dY set to the
    E5M2 Inf / NaN codes: those columns saturate / become NaN, amax (NaN ignored) becomes Inf."""
    rng = np.random.default_rng(3)
    m, n, k = 256, 256, 8192
    W = oracle.encode(E4, (rng.standard_normal(m * k) * 0.02 * 64).astype(np.float32))
    dY = oracle.encode(E5, (rng.standard_normal(k * n) * 1e-3 * 1024).astype(np.float32))
    hit = rng.choice(k * n, max(2, k * n // 100000), replace=False)
    dY[hit] = rng.choice(np.array([0x7C, 0xFC, 0x7D, 0x7E, 0x7F, 0xFF], np.uint8), hit.size)
    case = gu.GemmCase(None, 0, 0, m, n, k, E4, E5, ddt=E5, sa=1 / 64, sb=1 / 1024, qscale=4.0, amax=True, pad=0,
                       A=W, B=dY)
    s, D, amax = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first
    assert amax == np.inf


# ---- the BF16-matrix-core kernel: FP8 x FP8 with k < 8192 (k a multiple of 256) in every layout, and
# FP8 x K-contiguous BF16 (k a multiple of 128); FP8 widened exactly to BF16 per MFMA step ----------
@pytest.mark.parametrize("adt,bdt", [(E5, E4), (E4, E5), (E5, E5)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_h_fast_fp8_layouts(dev, ta, tb, adt, bdt):
    rng = np.random.default_rng(ta * 4 + tb * 2 + adt * 7 + bdt + 9100)
    case = gu.GemmCase(rng, ta, tb, 272, 304, 1024, adt, bdt, ddt=B16, pad=32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt", [E5, E4])
@pytest.mark.parametrize("ta", [1, 0])
@pytest.mark.parametrize("k", [256, 2048])
def test_h_fast_fp8_x_bf16(dev, ta, adt, k):
    rng = np.random.default_rng(ta * 2 + adt * 3 + k + 9200)
    case = gu.GemmCase(rng, ta, 0, 336, 272, k, adt, B16, ddt=B16, pad=16, dist="normal", sigma=3.0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb,bdt", [(1, 0, B16), (0, 0, B16), (0, 1, E4), (1, 1, E5)])
def test_h_fast_full_epilogue(dev, ta, tb, bdt):
    """OUTER scale vectors (FP8 operands), alpha, bias, beta * C of another dtype, FP32 output."""
    rng = np.random.default_rng(ta * 2 + tb + bdt + 9300)
    m, n = 288, 160
    sa = rng.uniform(0.25, 2.0, m).astype(np.float32)
    sb = rng.uniform(0.25, 2.0, n).astype(np.float32) if bdt != B16 else None
    case = gu.GemmCase(rng, ta, tb, m, n, 512, E4, bdt, ddt=F32, alpha=0.75, sa=sa, sb=sb, biasdt=F16, beta=0.5,
                       cdt=B16)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ta,tb,bdt", [(1, 0, B16), (0, 0, E5), (0, 1, E4)])
def test_h_fast_fp8_output(dev, ta, tb, bdt):
    rng = np.random.default_rng(ta * 2 + tb + bdt + 9400)
    case = gu.GemmCase(rng, ta, tb, 256, 512, 1024, E5, bdt, ddt=E4, qscale=0.25, amax=True, sa=0.5, pad=0,
                       dist="normal", sigma=2.0)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


def test_h_fast_inf_nan_operands(dev):
    """E5M2 Inf / NaN codes widen to BF16 Inf / NaN: saturated / NaN outputs and an Inf amax."""
    rng = np.random.default_rng(9500)
    m, n, k = 256, 256, 512
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, B16, ddt=E5, qscale=1.0, amax=True, pad=0, dist="normal", sigma=0.5)
    A = case.A.copy()
    A[3 * k + 5] = 0x7C   # +Inf in row 3
    A[77 * k + 9] = 0xFC  # -Inf in row 77
    A[150 * k + 1] = 0x7E  # NaN in row 150
    case.A = A
    s, D, amax = case.run(dev)
    assert s == 0
    bad, first = case.check(D)
    assert bad == 0, first
    assert amax == np.inf


def test_h_config3_fp8_x_bf16_sampled(dev):
    """Config 3's second GEMM (E5M2 A x BF16 B, N(0,1) * 8 values, scale_inv 1/64 on A) at k = 8192 on a
    2048 x 2048 output, sampled check."""
    rng = np.random.default_rng(9600)
    case = gu.GemmCase(rng, 1, 0, 2048, 2048, 8192, E5, B16, ddt=B16, dist="normal", sigma=8.0, sa=1 / 64, pad=0)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


# ---- split-K (e5ma_gemm_ex with a caller workspace): outputs with at most a quarter as many 256 x 256
# tiles as CUs split K into FP32 partials that a reduce kernel sums in order and runs through the
# epilogue; e5ma_gemm never splits.  These check the unsplit kernels (more than 64 tiles) and split
# counts at the edges ---------------------------------------------------------------------------------
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 0)])
def test_fast_unsplit_f8_sampled(dev, ta, tb):
    rng = np.random.default_rng(9700 + ta * 2 + tb)
    case = gu.GemmCase(rng, ta, tb, 4096, 4096, 8192, E5, E4, ddt=B16, dist="normal", sigma=8.0, sa=1 / 64,
                       sb=1 / 64, pad=0)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


def test_fast_unsplit_h_sampled(dev):
    rng = np.random.default_rng(9800)
    case = gu.GemmCase(rng, 1, 0, 4096, 3072, 1024, E4, B16, ddt=F32, dist="normal", sigma=2.0, sa=0.5, pad=0,
                       biasdt=F32, beta=0.5, cdt=B16)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("k,ta,tb,ddt", [(8192, 1, 0, B16), (8192, 0, 1, F32), (1024, 1, 0, B16), (1024, 0, 0, F32)])
def test_persistent_partial_last_round(dev, k, ta, tb, ddt):
    """4608 x 4352 = 18 x 17 = 306 tiles on a persistent grid of one block per CU: 50 blocks take two tiles
    and the other blocks, with no tile in the last round, start late.  FP8 matrix cores (k = 8192) and BF16
    ones (k = 1024); the BF16 write-out and the full one (FP32 D, bias, beta * BF16 C); sampled against the
    oracle's bound, the padding rows of D untouched."""
    rng = np.random.default_rng(9900 + k + 2 * ta + tb + ddt)
    kw = dict(biasdt=F32, beta=0.5, cdt=B16) if ddt == F32 else {}
    case = gu.GemmCase(rng, ta, tb, 4608, 4352, k, E5, E4, ddt=ddt, dist="normal", sigma=2.0, sa=0.5, sb=0.25,
                       pad=0, ldd=4608 + 8, **kw)
    bad, first = case.run_and_check(dev, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("m,n,k,adt,bdt", [(8192, 32, 8192, E5, E4), (256, 256, 16384, E4, E5),
                                            (1024, 8192, 8192, E5, E5), (64, 48, 512, E5, E4),
                                            (130, 20, 768, E4, B16)])
def test_splitk_shapes(dev, m, n, k, adt, bdt):
    """Skinny, tiny and half-filled grids through e5ma_gemm_ex with the workspace it asks for (split
    counts 8, 32, 1, 1 and 3 on 256 CUs), FP8 output with amax."""
    rng = np.random.default_rng(m + n + k)
    case = gu.GemmCase(rng, 1, 0, m, n, k, adt, bdt, ddt=E5, qscale=0.5, amax=True, dist="normal", sigma=2.0,
                       sa=0.25, pad=0 if m * n > 10**6 else 16)
    s, D, amax = case.run(dev, workspace="query")
    assert s == 0
    bad, first = case.check(D, amax, samples=4096 if m * n > 10**6 else None, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("m,n,k,adt,bdt,ta,tb", [(2048, 2048, 8192, E5, E4, 1, 0), (512, 768, 16384, E4, E5, 0, 1),
                                                  (1024, 512, 2048, E5, B16, 1, 0)])
def test_split_and_unsplit_both_in_bound(dev, m, n, k, adt, bdt, ta, tb):
    """The same GEMM unsplit (e5ma_gemm), split with the full workspace (e5ma_gemm_ex) and split fewer
    ways with a quarter of it: every result inside the oracle bound; a split sums the products in another
    order, so the bits may differ from the unsplit result's (they are not compared); the same split
    count gives the same bits on a repeat call (deterministic reduction)."""
    rng = np.random.default_rng(m + n + 3 * k)
    case = gu.GemmCase(rng, ta, tb, m, n, k, adt, bdt, ddt=F32, alpha=0.5, sa=0.25, biasdt=F32, beta=-0.5,
                       cdt=B16, dist="normal", sigma=2.0, pad=0)
    full = case.workspace_bytes()
    assert full > 0, "this shape splits K on a 256-CU device"
    results = []
    for ws in (None, full, full // 4):
        s, D, _ = case.run(dev, workspace=ws)
        assert s == 0
        bad, first = case.check(D, samples=4096, rng=rng)
        assert bad == 0, (ws, first)
        results.append(D)
    s, D2, _ = case.run(dev, workspace=full)
    assert s == 0 and np.array_equal(D2.view(np.uint32), results[1].view(np.uint32))


def test_workspace_query_matches_rule(dev):
    """e5ma_gemm_workspace_size: 0 for grids that fill more than a quarter of the CUs, for GEMV-routed
    calls and for the generic kernel; S * ldw * n * 4 bytes (ldw = m rounded up to 4) otherwise."""
    q = lambda ta, tb, m, n, k, a, b: gu._lib.workspace_size(ta, tb, m, n, k, a, k if ta else m, b, n if tb else k)
    assert q(1, 0, 8192, 8192, 8192, E5, E4) == 0
    assert q(1, 0, 8192, 4, 8192, E5, B16) == 0            # GEMV
    assert q(1, 0, 64, 64, 64, F32, F32) == 0              # generic kernel
    b = q(1, 0, 2048, 2048, 8192, E5, E4)
    assert b > 0 and b % (2048 * 2048 * 4) == 0 and b <= 64 << 20


def test_direct_epilogue_bf16_nan_codes(dev):
    """The direct epilogue's hardware BF16 conversion keeps a NaN's sign and payload; every NaN output
    must still be 0x7FC0.  Unsplit grid (81 tiles), BF16 output, no bias, beta = 0: NaN (0x7F, 0xFE) and
    Inf (0x7C) codes of A make rows 5, 6 NaN and row 9 Inf or NaN; sampled oracle check elsewhere."""
    rng = np.random.default_rng(9900)
    m = n = 2304
    k = 1024
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, B16, ddt=B16, dist="normal", sigma=1.0, pad=0, ldd=m + 4)
    A = case.A.copy()
    A[5 * k + 7] = 0x7F   # NaN
    A[6 * k + 3] = 0xFE   # negative NaN
    A[9 * k + 1] = 0x7C   # +Inf
    case.A = A
    s, D, _ = case.run(dev)
    assert s == 0
    Dm = D.view(np.uint16).reshape(n, case.ldd)[:, :m]
    assert (Dm[:, 5] == 0x7FC0).all() and (Dm[:, 6] == 0x7FC0).all()
    r9 = Dm[:, 9]
    assert (((r9 & 0x7FFF) == 0x7F80) | (r9 == 0x7FC0)).all()
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("k", [8192, 1024])
@pytest.mark.parametrize("m,n", [(2304, 2048), (2264, 2056)])
@pytest.mark.parametrize("vec", [False, True])
def test_staged16_bf16_nan_codes(dev, k, m, n, vec):
    """The 2-byte write-out (BF16 D, no bias, beta = 0, no amax, ldd % 8 == 0, m % 8 == 0) in each of its
    copies: full tiles (2304 x 2048) and edge tiles (2264 x 2056), per-tensor and per-row / per-column
    scales, on the FP8 (k = 8192) and the BF16 (k = 1024) matrix cores.  NaN codes of A make rows 5 and 6
    NaN, which must come out as 0x7FC0 (the screen over the converted pairs sets the block's flag); an Inf
    code makes row 9 Inf or NaN; sampled outputs elsewhere against the oracle's bound."""
    rng = np.random.default_rng(9950 + k + m + 3 * vec)
    sa = (rng.uniform(0.5, 2.0, m).astype(np.float32) / 64) if vec else 1.0 / 64
    sb = rng.uniform(0.5, 2.0, n).astype(np.float32) if vec else 0.5
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, E4, ddt=B16, sa=sa, sb=sb, dist="normal", sigma=1.0, pad=0,
                       ldd=m + 8)
    A = case.A.copy()
    A[5 * k + 7] = 0x7F   # NaN
    A[6 * k + 3] = 0xFE   # negative NaN
    A[9 * k + 1] = 0x7C   # +Inf
    case.A = A
    s, D, _ = case.run(dev)
    assert s == 0, gu._lib.last_error()
    Dm = D.view(np.uint16).reshape(n, case.ldd)[:, :m]
    assert (Dm[:, 5] == 0x7FC0).all() and (Dm[:, 6] == 0x7FC0).all()
    r9 = Dm[:, 9]
    assert (((r9 & 0x7FFF) == 0x7F80) | (r9 == 0x7FC0)).all()
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


# ---- the direct epilogue (full tiles, no bias, beta = 0, D columns 16-byte aligned: ldd % 4 == 0) on
# unsplit grids (more than 64 tiles), every output dtype, outer scales, amax ---------------------------
@pytest.mark.parametrize("ddt", [B16, F16, F32, E5, E4])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_epilogue_f8(dev, ta, tb, ddt):
    rng = np.random.default_rng(10000 + ta * 2 + tb + 10 * ddt)
    m, n, k = 2304, 2048, 8192
    sa = rng.uniform(0.5, 2.0, m).astype(np.float32) * (1 / 64)
    sb = rng.uniform(0.5, 2.0, n).astype(np.float32) * (1 / 64)
    case = gu.GemmCase(rng, ta, tb, m, n, k, E5, E4, ddt=ddt, alpha=0.5, sa=sa, sb=sb, dist="normal", sigma=8.0,
                       pad=0, ldd=m + 4, amax=True, qscale=0.25 if ddt in (E5, E4) else None)
    s, D, amax = case.run(dev)
    assert s == 0
    bad, first = case.check(D, amax, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("bdt", [B16, E5])
def test_direct_epilogue_h(dev, bdt):
    rng = np.random.default_rng(10100 + bdt)
    m, n, k = 2304, 2304, 1024
    case = gu.GemmCase(rng, 1, 0, m, n, k, E4, bdt, ddt=B16, sa=0.5, sb=0.25 if bdt == E5 else None,
                       dist="normal", sigma=2.0, pad=0, ldd=m + 4)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


# ---- the direct epilogue with a bias and / or beta * FP32 C (full tiles, D and C columns 16-byte aligned)
# on unsplit grids: TE's wgrad into main_grad (C = NULL, beta = 1), a separate C, linear layers with a bias
@pytest.mark.parametrize("mode,ddt", [("bias", B16), ("bias", E5), ("acc", F32), ("acc_bias", F32), ("c_bias", F32),
                                      ("c", B16)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_general_epilogue_f8(dev, ta, tb, mode, ddt):
    rng = np.random.default_rng(10200 + ta * 2 + tb + 10 * ddt + len(mode))
    m, n, k = 2304, 2048, 8192
    sa = rng.uniform(0.5, 2.0, m).astype(np.float32) * (1 / 64)
    sb = rng.uniform(0.5, 2.0, n).astype(np.float32) * (1 / 64)
    beta = 0.0 if mode == "bias" else 1.0 if mode.startswith("acc") else -0.5
    case = gu.GemmCase(rng, ta, tb, m, n, k, E5, E4, ddt=ddt, alpha=0.5, sa=sa, sb=sb, beta=beta,
                       cdt=F32 if mode.startswith("c") else None, biasdt=(B16 if ddt != F32 else F32) if "bias" in mode
                       else None, dist="normal", sigma=8.0, pad=0, ldd=m + 4, ldc=m + 8, amax=True,
                       qscale=0.25 if ddt in (E5, E4) else None)
    s, D, amax = case.run(dev)
    assert s == 0
    bad, first = case.check(D, amax, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("mode", ["acc_bias", "c"])
def test_direct_general_epilogue_h(dev, mode):
    rng = np.random.default_rng(10300 + len(mode))
    m, n, k = 2304, 2304, 1024
    case = gu.GemmCase(rng, 1, 0, m, n, k, E4, B16, ddt=F32, sa=0.5, beta=1.0 if mode == "acc_bias" else 0.25,
                       cdt=None if mode == "acc_bias" else F32, biasdt=F32 if mode == "acc_bias" else None,
                       dist="normal", sigma=2.0, pad=0, ldd=m + 4, ldc=m + 4)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first
