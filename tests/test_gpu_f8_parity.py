"""Parity of the FP8 matrix-core GEMM path (gemm_f8_kernel: v_mfma_f32_32x32x64_f8f6f4, every FP8 x FP8
call with k >= 8192) at the BASELINE shapes, on unsplit grids.

* Exact products: every finite code pair of every pairing, subnormals included, as the only non-zero
  term of its output at k = 8192, in all four layouts: D (FP32) == a * b bit for bit (the reference's
  exhaustive MAC check, tests/test_e5m2effma.cu:29-37,69-79, restated for one MAC per output).
* Config 3 (8192^3, E5M2 x E5M2 and E5M2 x E4M3 -> BF16, 0.01 % of the entries 57344, scale_inv 1/64):
  4096 sampled outputs against the oracle bound (reference shapes tests/test_gemm.cu:26-31).
* Config 4 at its own shapes: TE dgrad (N, N), both wgrad forms into an FP32 main_grad with bias and
  beta = 1, and run 3 (E5M2 output, scale, amax, 0.001 % Inf / NaN codes in dY).
* The documented accumulation deviation of the FP8 matrix cores (products below 2^(E-13) of their group's
  largest are truncated), pinned so that a change of hardware or compiler behaviour is noticed.
"""
import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
E5, E4, B16, F32 = oracle.E5M2, oracle.E4M3, oracle.BF16, oracle.FP32
LAYOUTS = [(1, 0), (0, 0), (0, 1), (1, 1)]


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def finite_codes(fmt):
    """All 256 codes, the Inf / NaN ones replaced by 0 (outside the operand contract)."""
    c = np.arange(256, dtype=np.uint8)
    bad = (c & 0x7C) == 0x7C if fmt == E5 else (c & 0x7F) == 0x7F
    c[bad] = 0
    return c


def store(mat_rk, contiguous_k, ld):
    """Lay out a logical [rows][k] matrix as the C ABI reads it: K-contiguous rows (ld >= k) or
    k-rows of `rows` contiguous elements (ld >= rows)."""
    rows, k = mat_rk.shape
    if contiguous_k:
        out = np.zeros((rows, ld), mat_rk.dtype)
        out[:, :k] = mat_rk
    else:
        out = np.zeros((k, ld), mat_rk.dtype)
        out[:, :rows] = mat_rk.T
    return out.ravel()


@pytest.mark.parametrize("adt,bdt", [(E5, E5), (E5, E4), (E4, E5), (E4, E4)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_f8_path_every_code_pair_exact(dev, ta, tb, adt, bdt):
    """m = 2304 (9 row tiles), n = 2048, k = 8192: 72 tiles, so one unsplit launch of the FP8 kernel.
    Row i carries code i % 256 at k0(i // 256), column j code j % 256 at every k0(t); all other entries
    are zero, so output (i, j) holds exactly one product, code(i % 256) * code(j % 256), at k0 spread
    over the whole K range.  Covers all 65536 pairs of the pairing 72 / 4 = 18 times over the tiles."""
    m, n, k = 2304, 2048, 8192
    k0 = (np.arange(m // 256) * 911 + 37) % k
    ca, cb = finite_codes(adt), finite_codes(bdt)
    A = np.zeros((m, k), np.uint8)
    A[np.arange(m), k0[np.arange(m) // 256]] = ca[np.arange(m) % 256]
    B = np.zeros((n, k), np.uint8)
    for t in k0:
        B[:, t] = cb[np.arange(n) % 256]
    lda = k if ta else m
    ldb = k if not tb else n
    case = gu.GemmCase(None, ta, tb, m, n, k, adt, bdt, ddt=F32, pad=0, A=store(A, ta == 1, lda),
                       B=store(B, tb == 0, ldb), ldd=m)
    assert case.lda == lda and case.ldb == ldb
    s, D, _ = case.run(dev)
    assert s == 0
    va = oracle.decode(adt, ca[np.arange(m) % 256]).astype(np.float64)
    vb = oracle.decode(bdt, cb[np.arange(n) % 256]).astype(np.float64)
    want = np.outer(vb, va).astype(np.float32)  # [j][i]; products of two FP8 values are exact in FP32
    got = D.reshape(n, m)
    # compared as values: the accumulator starts at +0, so a -0 product reads +0
    diff = np.nonzero(got != want)
    assert diff[0].size == 0, (diff[0].size, [(int(i), int(j), float(got[j, i]), float(want[j, i]))
                                              for j, i in zip(diff[0][:4], diff[1][:4])])


def config3_operands(rng, n_elem, fmt):
    """N(0, 1) * 8 values, 0.01 % of them replaced by the largest finite value 57344, encoded RNE
    satfinite."""
    x = rng.standard_normal(n_elem, dtype=np.float32) * np.float32(8.0)
    x[rng.integers(0, n_elem, n_elem // 10000)] = 57344.0
    return oracle.encode(fmt, x)


@pytest.mark.parametrize("bdt", [E5, E4])
def test_config3_8192_cube_sampled(dev, bdt):
    """8192^3 TN, A E5M2, B E5M2 (config 3) or E4M3 (the headline pairing), scale_inv 1/64 each,
    alpha 1, beta 0, BF16 D with ldd = m (the direct epilogue the benchmark times)."""
    rng = np.random.default_rng(0xE5A003 + bdt)
    m = n = k = 8192
    A = config3_operands(rng, m * k, E5)
    B = config3_operands(rng, n * k, bdt)
    assert np.count_nonzero(A == 0x7B) >= m * k // 10000 // 2
    case = gu.GemmCase(None, 1, 0, m, n, k, E5, bdt, ddt=B16, sa=1 / 64, sb=1 / 64, pad=0, A=A, B=B, ldd=m)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first
    # the outputs of rows holding saturated entries are checked too
    sat_rows = np.unique(np.nonzero(A == 0x7B)[0] // k)[:512]
    iis = np.repeat(sat_rows, 8)
    jjs = rng.integers(0, n, iis.size)
    bad2, first2, _, _ = case.oracle_gemm().check(D, None, iis, jjs)
    assert bad2 == 0, first2


TOK, HID, FFN = 8192, 4096, 14336


def te_operands(rng):
    W = oracle.encode(E4, rng.standard_normal(FFN * HID, dtype=np.float32) * np.float32(0.02 * 64))
    dY = oracle.encode(E5, rng.standard_normal(TOK * FFN, dtype=np.float32) * np.float32(1e-3 * 1024))
    return W, dY


def test_config4_dgrad_full_shape(dev):
    """dX^T [hid, tok] = W^T dY^T: e5ma_gemm(N, N, 4096, 8192, 14336), A = W [ffn][hid] E4M3 (lda = hid),
    B = dY [tok][ffn] E5M2 (ldb = ffn), row-wise scale_inv vectors of both, BF16 out."""
    rng = np.random.default_rng(0xE5A004)
    W, dY = te_operands(rng)
    sa = (np.full(HID, 1 / 64) * rng.uniform(0.5, 2, HID)).astype(np.float32)
    sb = (np.full(TOK, 1 / 1024) * rng.uniform(0.5, 2, TOK)).astype(np.float32)
    case = gu.GemmCase(None, 0, 0, HID, TOK, FFN, E4, E5, ddt=B16, sa=sa, sb=sb, pad=0, A=W, B=dY, ldd=HID)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


@pytest.mark.parametrize("form", ["NT", "TN"])
def test_config4_wgrad_full_shape(dev, form):
    """main_grad += dY^T X + bias with beta = 1 and C = NULL (TE accumulate), FP32 D:
    NT: e5ma_gemm(N, T, ffn, hid, tok), A = dY [tok][ffn] (lda = ffn), B = X [tok][hid] (ldb = hid);
    TN: from token-contiguous copies, e5ma_gemm(T, N, hid, ffn, tok), A = X^T storage [hid][tok],
        B = dY^T storage [ffn][tok] (the same values, transposed storage)."""
    rng = np.random.default_rng(0xE5A005 + len(form))
    dY = oracle.encode(E5, rng.standard_normal(TOK * FFN, dtype=np.float32) * np.float32(1e-3 * 1024))
    X = oracle.encode(E4, rng.standard_normal(TOK * HID, dtype=np.float32) * np.float32(2.0))
    if form == "NT":
        m, n, ta, tb, A, B, adt, bdt, sa, sb = FFN, HID, 0, 1, dY, X, E5, E4, 1 / 1024, 0.5
    else:
        m, n, ta, tb, adt, bdt, sa, sb = HID, FFN, 1, 0, E4, E5, 0.5, 1 / 1024
        A = X.reshape(TOK, HID).T.copy().ravel()
        B = dY.reshape(TOK, FFN).T.copy().ravel()
    D0 = rng.uniform(-1, 1, m * n).astype(np.float32)
    case = gu.GemmCase(rng, ta, tb, m, n, TOK, adt, bdt, ddt=F32, sa=sa, sb=sb, beta=1.0, biasdt=F32, pad=0, A=A,
                       B=B, D0=D0, ldd=m)
    s, D, _ = case.run(dev)
    assert s == 0
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first


def test_config4_run3_e5m2_output_inf_nan_full_shape(dev):
    """dgrad shape with E5M2 output (scale 4, amax) and 0.001 % of dY set to the E5M2 Inf / NaN codes:
    outputs of the columns they reach are saturated or NaN (0x7F), amax (NaN ignored) is Inf."""
    rng = np.random.default_rng(0xE5A006)
    W, dY = te_operands(rng)
    hit = rng.choice(dY.size, dY.size // 100000, replace=False)
    dY[hit] = rng.choice(np.array([0x7C, 0xFC, 0x7D, 0x7E, 0x7F, 0xFF], np.uint8), hit.size)
    sa = np.full(HID, 1 / 64, np.float32)
    sb = np.full(TOK, 1 / 1024, np.float32)
    case = gu.GemmCase(None, 0, 0, HID, TOK, FFN, E4, E5, ddt=E5, sa=sa, sb=sb, qscale=4.0, amax=True, pad=0, A=W,
                       B=dY, ldd=HID)
    s, D, amax = case.run(dev)
    assert s == 0
    assert amax == np.inf
    # every column of dY^T holding a NaN code yields NaN in all of its outputs
    nan_cols = np.unique(hit[np.isin(dY[hit], [0x7D, 0x7E, 0x7F, 0xFF])] // FFN)
    Dm = D.reshape(TOK, HID)
    assert (Dm[nan_cols] == 0x7F).all()
    bad, first = case.check(D, samples=4096, rng=rng)
    assert bad == 0, first
    # and outputs the special codes reach are checked too: sample them explicitly
    cols = np.unique(hit // FFN)[:64]
    iis = rng.integers(0, HID, cols.size * 8)
    jjs = np.repeat(cols, 8)
    g = case.oracle_gemm()
    bad2, first2, _, _ = g.check(D, None, iis, jjs)
    assert bad2 == 0, first2


# ---- the accumulation deviation of the FP8 matrix cores, pinned -----------------------------------
def _one_group(dev, prods_at):
    """A 256 x 256 x 8192 TN E5M2 x E5M2 GEMM whose every output has the products prods_at (list of
    (k, value of a, value of b)), all other terms zero; returns D (FP32) of output (0, 0)."""
    m = n = 256
    k = 8192
    A = np.zeros((m, k), np.uint8)
    B = np.zeros((n, k), np.uint8)
    for kk, va, vb in prods_at:
        A[:, kk] = oracle.encode(E5, np.float32([va]))[0]
        B[:, kk] = oracle.encode(E5, np.float32([vb]))[0]
    case = gu.GemmCase(None, 1, 0, m, n, k, E5, E5, ddt=F32, pad=0, A=A.ravel(), B=B.ravel(), ldd=m)
    s, D, _ = case.run(dev)
    assert s == 0
    vals = D.reshape(n, m)
    assert (vals == vals[0, 0]).all()
    return float(vals[0, 0])


def test_f8_truncation_within_group_of_8(dev):
    """The FP8 matrix cores align the products of each group of 8 consecutive k to the group's largest
    exponent E and truncate them toward zero to multiples of 2^(E-13) (the deviation from exact products
    that INTEGRATION lists; it stays inside the contract bound for k >= 7646).  Pinned on a single
    group: 1 + 1.5 * 2^-14 (same group) reads 1; 1 + 1.5 * 2^-13 reads 1 + 2^-13; the same small
    product in another group of 8 is kept exactly."""
    small = 1.5 * 2.0**-14
    assert _one_group(dev, [(8, 1.0, 1.0), (9, small, 1.0)]) == 1.0
    assert _one_group(dev, [(8, 1.0, 1.0), (12, 2 * small, 1.0)]) == 1.0 + 2.0**-13
    assert _one_group(dev, [(8, 1.0, 1.0), (16, small, 1.0)]) == 1.0 + small
