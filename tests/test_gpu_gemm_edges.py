"""Edge tiles of the fast GEMM kernels against the oracle's bound: m and n that are not multiples of the
256 x 256 block tile, through each write-out class:
- m % 8 == 0, 2-byte D, no bias, beta = 0: the staged 2-byte write-out (stores per 8 rows, columns past n
  skipped);
- m % 4 == 0 (or bias / beta * C / FP32 or FP8 D): the staged general write-out (4-row groups);
- odd m or unaligned D: the half-tile write-out with per-element bounds checks.
Every output is checked (and amax, where asked), and the rows between m and ldd of every column of D must
stay untouched.  k = 8192 runs the FP8 matrix cores, k = 512 the BF16 ones (FP8 x FP8 with short k);
the reference's tail cases are tests/test_gemm.cu:13-46 (m / n not multiples of its tile)."""
import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
E5, E4, B16, F32 = oracle.E5M2, oracle.E4M3, oracle.BF16, oracle.FP32


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


# (m, n): m % 8 == 0; m % 4 == 0 only; odd m; an n edge only; m and n multiples of 16 (the fast kernels'
# M / N-contiguous layouts need that; other shapes of those layouts run the generic kernel)
SHAPES = [(264, 272), (260, 272), (262, 272), (512, 280), (272, 304)]


@pytest.mark.parametrize("m,n", SHAPES)
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 1)])
@pytest.mark.parametrize("k", [8192, 512])
def test_edges_bf16_out(dev, m, n, ta, tb, k):
    rng = np.random.default_rng(m * 31 + n + 7 * ta + k)
    case = gu.GemmCase(rng, ta, tb, m, n, k, E5, E4, ddt=B16, sa=0.5, sb=0.25, dist="normal", sigma=2.0, pad=0,
                       ldd=m + 8)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("m,n", SHAPES)
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 0)])
def test_edges_fp32_accumulate_with_bias_and_row_scales(dev, m, n, ta, tb):
    """TE wgrad's epilogue at edge tiles: alpha, per-row and per-column scale_inv, bias, beta * FP32 C, amax."""
    rng = np.random.default_rng(m * 13 + n + ta + 5 * tb)
    sa = (0.25 + rng.integers(0, 64, m) / 64).astype(np.float32)
    sb = (0.25 + rng.integers(0, 64, n) / 64).astype(np.float32)
    case = gu.GemmCase(rng, ta, tb, m, n, 8192, E5, E4, ddt=F32, alpha=0.75, sa=sa, sb=sb, beta=1.0, cdt=F32,
                       biasdt=F32, amax=True, dist="normal", sigma=2.0, pad=0, ldd=m + 4, ldc=m + 8)
    s, D, amax = case.run(dev)
    assert s == 0, gu._lib.last_error()
    bad, first = case.check(D, amax)
    assert bad == 0, first


@pytest.mark.parametrize("m,n", [(264, 272), (262, 272)])
@pytest.mark.parametrize("ddt", [E5, E4])
def test_edges_fp8_out_amax(dev, m, n, ddt):
    rng = np.random.default_rng(m + n + ddt)
    case = gu.GemmCase(rng, 1, 0, m, n, 8192, E5, E4, ddt=ddt, sa=0.5, qscale=0.25, amax=True, dist="normal",
                       sigma=2.0, pad=0, ldd=m + 8)
    s, D, amax = case.run(dev)
    assert s == 0, gu._lib.last_error()
    bad, first = case.check(D, amax)
    assert bad == 0, first


@pytest.mark.parametrize("m,n,k", [(2000, 1808, 8192), (8000, 600, 8192)])
def test_edges_large_sampled(dev, m, n, k):
    """Many edge tiles at once (every round holds some), sampled outputs, padding rows checked whole."""
    rng = np.random.default_rng(m + n)
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, E4, ddt=B16, sa=1.0 / 64, sb=1.0 / 64, dist="normal", sigma=8.0,
                       pad=0, ldd=m + 8)
    bad, first = case.run_and_check(dev, samples=20000, rng=rng)
    assert bad == 0, first


def test_edge_results_do_not_depend_on_the_grid(dev):
    """A 520 x 528 GEMM equals the top-left corner of the 768 x 768 GEMM of the same operands bit for bit
    (each output's sum runs in the same order whatever the tile is: edge or full)."""
    rng = np.random.default_rng(77)
    k = 8192
    big = gu.GemmCase(rng, 1, 0, 768, 768, k, E5, E4, ddt=B16, sa=0.5, dist="normal", sigma=2.0, pad=0, ldd=768)
    s, Dbig, _ = big.run(dev)
    assert s == 0
    # the same A rows / B columns, cut to 520 x 528 (TN: A is m x k row-major, B is n x k row-major)
    A = big.A.reshape(768, big.lda)[:520].ravel()
    B = big.B.reshape(768, big.ldb)[:528].ravel()
    small = gu.GemmCase(rng, 1, 0, 520, 528, k, E5, E4, ddt=B16, sa=0.5, pad=0, ldd=520, A=A, B=B)
    small.lda, small.ldb = big.lda, big.ldb
    s, Dsmall, _ = small.run(dev)
    assert s == 0
    want = Dbig.reshape(768, 768)[:528, :520]
    assert np.array_equal(Dsmall.reshape(528, 520).view(np.uint16), want.view(np.uint16))
