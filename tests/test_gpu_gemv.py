"""The GEMV path of e5ma_gemm (n <= 8, transa = T, transb = N, FP8 A; reference routing
src/gemm_e5m2effma.cu:100-102) against the oracle bound, mirroring tests/test_gemv.cu:12-21 (A in
{E5M2, E4M3} x x in four dtypes x n = 1..8, row-wise scales) plus exact single products and the
BASELINE config 2 shape."""
import itertools

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


@pytest.mark.parametrize("adt,bdt", list(itertools.product([E5, E4], [E5, E4, B16, F32])))
@pytest.mark.parametrize("n", range(1, 9))
def test_gemv_dtypes_and_widths(dev, adt, bdt, n):
    rng = np.random.default_rng(adt * 1000 + bdt * 100 + n)
    m, k = 300, 1040
    sa = (0.25 + rng.integers(0, 1024, m) / 512).astype(np.float32)
    sb = 0.75 if bdt in gu.FP8 else None
    case = gu.GemmCase(rng, 1, 0, m, n, k, adt, bdt, ddt=B16, alpha=1.5, sa=sa, sb=sb, biasdt=F32, amax=True)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("ddt", [F32, E4])
def test_gemv_epilogue(dev, ddt):
    rng = np.random.default_rng(ddt)
    qs = 2.0 if ddt == E4 else None
    case = gu.GemmCase(rng, 1, 0, 257, 3, 512, E5, E5, ddt=ddt, sa=0.5, sb=0.25, beta=0.5, cdt=B16, biasdt=B16,
                       qscale=qs, amax=True)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first
    acc = gu.GemmCase(rng, 1, 0, 100, 8, 256, E4, F32, ddt=F32, beta=1.0, cdt=None)
    bad, first = acc.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E4, E4), (E5, B16), (E4, F32)])
def test_gemv_single_product_exact(dev, adt, bdt):
    """One non-zero k per row: every A code times x is exact (FP32 output)."""
    m, k, n = 256, 32, 1
    a = np.arange(256, dtype=np.uint8)
    a[((a & 0x7C) == 0x7C) if adt == E5 else ((a & 0x7F) == 0x7F)] = 0
    A = np.zeros(m * k, np.uint8)
    A[np.arange(m) * k + 17] = a
    xv = np.float32(1.25) if bdt != E5 else np.float32(1.5)
    x = np.zeros(k, np.float32)
    x[17] = xv
    B = oracle.encode(bdt, x) if bdt != F32 else x
    case = gu.GemmCase(None, 1, 0, m, n, k, adt, bdt, ddt=F32, pad=0, A=A, B=B)
    s, D, _ = case.run(dev)
    assert s == 0
    want = (oracle.decode(adt, a).astype(np.float64) * float(oracle.decode(bdt, B)[17])).astype(np.float32)
    assert np.array_equal(D[:m], want)


@pytest.mark.parametrize("n", [1, 8])
def test_gemv_config2(dev, n):
    """BASELINE config 2 GEMV: W 8192 x 8192 E5M2 from N(0, 0.02) with a row-wise scale_inv, x BF16
    N(0, 1), batch 1 and 8, BF16 output; every output checked."""
    rng = np.random.default_rng(0xE5A002 + n)
    m = k = 8192
    w = rng.standard_normal(m * k, dtype=np.float32) * np.float32(0.02)
    amax = np.abs(w).max()
    A = oracle.encode(E5, w, float(np.float32(57344.0) / amax))
    sa = np.full(m, amax / np.float32(57344.0), np.float32)
    x = oracle.encode(B16, rng.standard_normal(k * n).astype(np.float32))
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, B16, ddt=B16, sa=sa, pad=0, A=A, B=x)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


# ---- the matrix-core kernel (n = 5 .. 8 with a BF16 or FP8 x) ------------------------------------
@pytest.mark.parametrize("n", [5, 8])
@pytest.mark.parametrize("ddt", [F32, E4, E5])
def test_gemv_mfma_epilogue(dev, n, ddt):
    """alpha, row-wise and per-tensor scale_inv, bias, beta * C (BF16), FP8 output with scale and amax,
    on m and k that leave partial row groups and partial batches."""
    rng = np.random.default_rng(7000 + 10 * n + ddt)
    m, k = 203, 2064
    qs = 0.5 if ddt in gu.FP8 else None
    sa = (0.25 + rng.integers(0, 1024, m) / 512).astype(np.float32)
    case = gu.GemmCase(rng, 1, 0, m, n, k, E5, E4, ddt=ddt, alpha=0.75, sa=sa, sb=0.5, beta=0.5, cdt=B16,
                       biasdt=B16, qscale=qs, amax=True)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("n,bdt", [(6, B16), (7, E5)])
def test_gemv_mfma_accumulate(dev, n, bdt):
    """TE accumulate on the matrix-core kernel: C = NULL, beta = 1 reads and writes D (FP32)."""
    rng = np.random.default_rng(7100 + n)
    case = gu.GemmCase(rng, 1, 0, 160, n, 1040, E4, bdt, ddt=F32, beta=1.0, cdt=None, biasdt=F32)
    bad, first = case.run_and_check(dev)
    assert bad == 0, first


@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E4, E4), (E5, B16), (E4, B16)])
def test_gemv_mfma_single_product_exact(dev, adt, bdt):
    """n = 8, one non-zero k per row: every finite A code times x is exact through the BF16 widening and
    the matrix-core accumulation (FP32 output); every column gets its own x value."""
    m, k, n = 256, 64, 8
    a = np.arange(256, dtype=np.uint8)
    a[((a & 0x7C) == 0x7C) if adt == E5 else ((a & 0x7F) == 0x7F)] = 0
    A = np.zeros(m * k, np.uint8)
    A[np.arange(m) * k + 41] = a
    x = np.zeros(k * n, np.float32)
    xs = np.array([1.25, -1.5, 0.75, 2.0, -0.5, 1.75, 3.0, -2.5], np.float32)
    x[np.arange(n) * k + 41] = xs
    B = oracle.encode(bdt, x)
    case = gu.GemmCase(None, 1, 0, m, n, k, adt, bdt, ddt=F32, pad=0, A=A, B=B)
    s, D, _ = case.run(dev)
    assert s == 0
    xd = oracle.decode(bdt, B).reshape(n, k)[:, 41].astype(np.float64)
    for j in range(n):
        want = (oracle.decode(adt, a).astype(np.float64) * xd[j]).astype(np.float32)
        assert np.array_equal(D[j * case.ldd: j * case.ldd + m], want), j


def test_gemv_mfma_deterministic(dev):
    """Two calls on the same inputs give identical bits (wave partials are summed in a fixed order)."""
    rng = np.random.default_rng(7200)
    case = gu.GemmCase(rng, 1, 0, 512, 8, 4096, E5, B16, ddt=F32, sa=0.5)
    s1, D1, _ = case.run(dev)
    s2, D2, _ = case.run(dev)
    assert s1 == 0 and s2 == 0
    assert np.array_equal(D1.view(np.uint32), D2.view(np.uint32))
