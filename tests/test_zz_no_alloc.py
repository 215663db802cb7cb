"""e5ma_gemm_noalloc (include/e5m2effma_ext.h): e5ma_gemm_ex on the library's fixed per-device scratch.
Called through the C ABI and compared bit for bit with e5ma_gemm_ex given the workspace
e5ma_gemm_workspace_size reports (same split count, same partials, same reduction order), on two calls in
a row, the second with a smaller input, so the second runs on scratch that still holds the first call's
partials; both are also held to the oracle bound.  A GEMV-routed call and an unsplit one (more tiles than
a quarter of the CUs) go through the same entry point unchanged."""
import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from e5m2effma_amd import _lib

pytestmark = pytest.mark.gpu
E5, E4, B16, F32 = oracle.E5M2, oracle.E4M3, oracle.BF16, oracle.FP32


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def run_noalloc(case, dev):
    """case through e5ma_gemm_noalloc; returns (status, D)."""
    keep = []

    def put(a):
        t, p = gu.to_dev(a, dev)
        keep.append(t)
        return p
    pa, pb = put(case.A), put(case.B)
    pbias = put(case.bias) if case.bias is not None else None
    pc = put(case.C) if case.C is not None else None
    Dt, pd = gu.to_dev(case.D0, dev)
    sa_t, sa_p = gu.dev_floats(case.sa, dev)
    sb_t, sb_p = gu.dev_floats(case.sb, dev)
    A = _lib.tensor(pa, case.adt, sa_p)
    B = _lib.tensor(pb, case.bdt, sb_p)
    C = _lib.tensor(pc, case.cdt) if pc is not None else None
    D = _lib.tensor(pd, case.ddt)
    bias = _lib.tensor(pbias, case.biasdt) if pbias is not None else None
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    s = _lib.lib().e5ma_gemm_noalloc(case.transa, case.transb, case.m, case.n, case.k, float(case.alpha), _lib.ref(A),
                                     case.lda, _lib.ref(B), case.ldb, float(case.beta), _lib.ref(C), case.ldc,
                                     _lib.ref(D), case.ldd, _lib.ref(bias), st)
    torch.cuda.synchronize(dev)
    return s, gu.from_dev(Dt, pd, gu.NPD[case.ddt], case.ldd * case.n)


def make(rng, m, n, k, adt, bdt, ddt=B16):
    return gu.GemmCase(rng, 1, 0, m, n, k, adt, bdt, ddt=ddt, alpha=0.75, sa=0.25, sb=0.5, biasdt=F32, beta=0.5,
                       cdt=B16, dist="normal", sigma=2.0, pad=0)


def test_noalloc_matches_gemm_ex_twice(dev):
    """2048^2 x 8192 (64 tiles: 4 splits, the whole 64 MiB scratch), then 512^2 x 8192 (4 tiles: 32 splits,
    half of it): each bit-identical to e5ma_gemm_ex with its queried workspace and inside the bound."""
    rng = np.random.default_rng(0xA110C)
    for m, n, k, adt, bdt in ((2048, 2048, 8192, E5, E4), (512, 512, 8192, E4, E5)):
        case = make(rng, m, n, k, adt, bdt)
        assert case.workspace_bytes() > 0, "this shape splits K on a 256-CU device"
        s, D_ex, _ = case.run(dev, workspace="query")
        assert s == 0, _lib.last_error()
        s, D_na = run_noalloc(case, dev)
        assert s == 0, _lib.last_error()
        assert np.array_equal(D_na.view(np.uint16), D_ex.view(np.uint16)), (m, n, k)
        bad, first = case.check(D_na, samples=4096, rng=rng)
        assert bad == 0, (m, n, k, first)


def test_noalloc_gemv_and_unsplit_calls(dev):
    """Calls that need no scratch: a GEMV-routed one (n = 4) and a grid of 81 tiles, equal to e5ma_gemm's."""
    rng = np.random.default_rng(0xA110D)
    for m, n, k, adt, bdt in ((4096, 4, 8192, E5, B16), (2304, 2304, 1024, E4, E5)):
        case = make(rng, m, n, k, adt, bdt, ddt=F32)
        s, D_ref, _ = case.run(dev)
        assert s == 0, _lib.last_error()
        s, D_na = run_noalloc(case, dev)
        assert s == 0, _lib.last_error()
        assert np.array_equal(D_na.view(np.uint32), D_ref.view(np.uint32)), (m, n, k)
