"""Pins the CPU oracle (oracle/e5ma_oracle.c) before anything is checked against it.

Each oracle function is held to something it does not compute itself:
  * the reference's own exact MAC model (golden digests + vectors in tests/golden/, and the model
    itself when oracle/_ref/libref.so was built from the reference sources);
  * an exact rational (Fraction) model written here;
  * independent codecs (torch's float8 / bfloat16 casts, numpy's float16 cast, a midpoint search);
  * closed forms (single-product GEMMs, Adam with unit moments) and the reference's KATs.
Negative controls plant a mistake in an oracle-side value and check the checker rejects it.
"""
import hashlib
import json
import os
from fractions import Fraction as Fr

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PAIRINGS = [(1, 1), (1, 0), (0, 1), (0, 0)]


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(GOLD, "lane_golden.json")) as f:
        meta = json.load(f)
    return meta, np.load(os.path.join(GOLD, "lane_golden.npz"))


# ---- the exact MAC model -------------------------------------------------------------------------
@pytest.mark.parametrize("fa,fb", PAIRINGS)
def test_lane_full_sweep_matches_reference_digest(orc, golden, fa, fb):
    meta, _ = golden
    out = orc.lane_sweep(np.array(meta["corpus"], np.uint16), fa, fb)
    assert hashlib.sha256(out.astype("<u2").tobytes()).hexdigest() == meta["sha256"][f"{fa}{fb}"]


@pytest.mark.parametrize("fa,fb", PAIRINGS)
def test_lane_matches_reference_vectors(orc, golden, fa, fb):
    _, z = golden
    t = f"{fa}{fb}"
    got = orc.lane(z[f"a_{t}"], z[f"b_{t}"], z[f"acc_{t}"], fa, fb)
    np.testing.assert_array_equal(got, z[f"out_{t}"])


@pytest.mark.parametrize("fa,fb", PAIRINGS)
def test_lane_against_reference_library(orc, fa, fb):
    ref = orc.ref_library()
    if ref is None:
        pytest.skip("oracle/_ref/libref.so not built (reference sources absent)")
    import ctypes
    accs = np.arange(0, 0x10000, 97, dtype=np.uint16)  # 676 accumulators x 65,536 pairs
    first = ctypes.c_uint32(0)
    bad = orc.lib().orc_lane_compare(ctypes.cast(ref.ref_lane, ctypes.c_void_p), orc._p(accs), accs.size, fa, fb,
                                     ctypes.byref(first))
    assert bad == 0, hex(first.value)


def _fp8_frac(code, fmt):
    s, c = code >> 7, code & 0x7F
    if fmt == 1:
        e, f = c >> 2, c & 3
        if e == 31:
            return None
        v = Fr(f, 4) * Fr(2) ** -14 if e == 0 else (1 + Fr(f, 4)) * Fr(2) ** (e - 15)
    else:
        e, f = c >> 3, c & 7
        if c == 0x7F:
            return None
        v = Fr(f, 8) * Fr(2) ** -6 if e == 0 else (1 + Fr(f, 8)) * Fr(2) ** (e - 7)
    return -v if s else v


def _bf16_frac(h):
    e, f = (h >> 7) & 0xFF, h & 0x7F
    v = Fr(f, 128) * Fr(2) ** -126 if e == 0 else (1 + Fr(f, 128)) * Fr(2) ** (e - 127)
    return -v if h >> 15 else v


def _rn_bf16(x):
    """Round a Fraction to BF16 bits by exact comparison with the neighbours (ties to even)."""
    if x == 0:
        return 0
    s = 0x8000 if x < 0 else 0
    a = -x if x < 0 else x
    lo, hi = 0, 0x7F80  # bits of finite non-negative BF16 values are ordered like the values
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if _bf16_frac(mid) <= a:
            lo = mid
        else:
            hi = mid
    vl = _bf16_frac(lo)
    vh = _bf16_frac(hi) if hi < 0x7F80 else Fr(2) ** 128  # Inf stands where 2^128 would be
    if a == vl:
        return s | lo
    mid = (vl + vh) / 2
    pick = lo if a < mid else hi if a > mid else (lo if lo % 2 == 0 else hi)
    return s | pick


@pytest.mark.parametrize("fa,fb", PAIRINGS)
def test_lane_against_fraction_model(orc, fa, fb):
    rng = np.random.default_rng(7 + fa * 2 + fb)
    a = rng.integers(0, 256, 3000).astype(np.uint8)
    b = rng.integers(0, 256, 3000).astype(np.uint8)
    acc = rng.integers(0, 0x7F80, 3000).astype(np.uint16) | (rng.integers(0, 2, 3000).astype(np.uint16) << 15)
    got = orc.lane(a, b, acc, fa, fb)
    for x, y, c, g in zip(a.tolist(), b.tolist(), acc.tolist(), got.tolist()):
        va, vb = _fp8_frac(x, fa), _fp8_frac(y, fb)
        if va is None or vb is None:
            assert g == 0x7FC0
            continue
        total = _bf16_frac(c) + va * vb
        if total == 0:
            both_neg_zero = va * vb == 0 and _bf16_frac(c) == 0 and (c >> 15) and ((x ^ y) >> 7)
            assert g == (0x8000 if both_neg_zero else 0)
        else:
            assert g == _rn_bf16(total), (hex(x), hex(y), hex(c))


# ---- codecs ----------------------------------------------------------------------------------------
@pytest.mark.parametrize("fmt,tdt", [(4, torch.float8_e5m2), (0, torch.float8_e4m3fn)])
def test_fp8_decode_all_codes_vs_torch(orc, fmt, tdt):
    codes = np.arange(256, dtype=np.uint8)
    got = orc.decode(fmt, codes)
    ref = torch.from_numpy(codes).view(tdt).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))  # bit equality: signed zeros too


def test_fp8_operand_decode_reads_special_codes_as_finite(orc):
    # reference src/e5m2effma.cuh:59-68 (E5M2 exponent-31 codes) and :43-52 (E4M3 0x7F -> 480)
    L = orc.lib()
    assert [L.orc_e5m2_operand(c) for c in (0x7C, 0x7D, 0x7E, 0x7F)] == [65536.0, 81920.0, 98304.0, 114688.0]
    assert L.orc_e4m3_operand(0x7F) == 480.0 and L.orc_e4m3_operand(0xFF) == -480.0
    for c in range(256):
        if (c & 0x7C) != 0x7C:
            assert L.orc_e5m2_operand(c) == L.orc_e5m2_value(c) or (c & 0x7F) == 0


@pytest.mark.parametrize("fmt", [4, 0])
def test_fp8_encoder_vs_midpoint_search(orc, fmt):
    import ctypes
    first = ctypes.c_uint32(0)
    L = orc.lib()
    # the whole 2^32 space at a prime stride, then every pattern of the FP8 range at a finer stride
    assert L.orc_encode_selfcheck(fmt, 0, 1 << 32, 65521, ctypes.byref(first)) == 0, hex(first.value)
    lo, hi = (0x37000000, 0x47800000) if fmt == 4 else (0x3B000000, 0x44000000)
    for sign in (0, 0x80000000):
        assert L.orc_encode_selfcheck(fmt, sign + lo, sign + hi, 509, ctypes.byref(first)) == 0, hex(first.value)


@pytest.mark.parametrize("fmt,tdt,top", [(4, torch.float8_e5m2, 57344.0), (0, torch.float8_e4m3fn, 448.0)])
def test_fp8_encoder_vs_torch_in_range(orc, fmt, tdt, top):
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 100.0)])
    x = np.concatenate([x, orc.decode(fmt, np.arange(256, dtype=np.uint8))])  # exact codes and midpoints
    vals = orc.decode(fmt, np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    x = np.concatenate([x, ((vals[:-1] + vals[1:]) / 2).astype(np.float32)])
    x = x[np.isfinite(x) & (np.abs(x) < top)]
    got = orc.encode(fmt, x)
    ref = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_fp8_encoder_kat(orc):
    # reference binds/python/tests/test_e5m2effma.py:122-125 (saturation as cvt.rn.satfinite)
    codes, amax = orc.cast(3, 4, np.array([1.0, np.inf, -1e6, 3.0], np.float32), 4)
    assert codes.tolist() == [0x3C, 0x7B, 0xFB, 0x42] and amax == np.inf
    nan = np.array([np.nan, -np.nan], np.float32)
    assert orc.encode(4, nan).tolist() == [0x7F, 0x7F] and orc.encode(0, nan).tolist() == [0x7F, 0x7F]
    assert orc.encode(0, np.array([448.0, 464.0, 1e9, -np.inf], np.float32)).tolist() == [0x7E, 0x7E, 0x7E, 0xFE]


def test_bf16_rne_vs_torch(orc):
    rng = np.random.default_rng(3)
    u = rng.integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    u = np.concatenate([u, np.arange(0x7F7F0000, 0x7F800000, 7, dtype=np.uint32),
                        (np.arange(0, 0x20000, dtype=np.uint32) | 0x3F800000)])  # overflow edge, all ties
    x = u.view(np.float32)
    got = orc.encode(1, x)
    isnan = np.isnan(x)
    assert (got[isnan] == 0x7FC0).all()
    ref = torch.from_numpy(x[~isnan]).to(torch.bfloat16).view(torch.uint16).numpy()
    assert np.array_equal(got[~isnan], ref)


def test_f16_rne_vs_numpy(orc):
    rng = np.random.default_rng(5)
    u = rng.integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    u = np.concatenate([u, np.arange(0x33000000, 0x47800000, 613, dtype=np.uint32)])  # the whole f16 range
    x = u.view(np.float32)
    got = orc.encode(2, x)
    isnan = np.isnan(x)
    assert np.isnan(orc.decode(2, got[isnan])).all()
    with np.errstate(over="ignore"):
        ref = x[~isnan].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[~isnan], ref)
    h = np.arange(0x10000, dtype=np.uint16)
    dec = orc.decode(2, h)
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(dec), np.isnan(ref)) and np.array_equal(dec[~np.isnan(ref)], ref[~np.isnan(ref)])


def test_cast_semantics(orc):
    """load * sinv, NaN-ignoring amax committed only when positive, store with qscale
    (reference src/e5m2effma.cu:53-63, src/e5m2effma.cuh:190-195)."""
    codes = np.arange(256, dtype=np.uint8)
    out, amax = orc.cast(4, 3, codes, 256, sinv=0.5)
    ref = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy() * np.float32(0.5)
    assert np.array_equal(np.isnan(out), np.isnan(ref)) and np.array_equal(out[~np.isnan(ref)], ref[~np.isnan(ref)])
    assert amax == np.inf  # Inf enters amax, NaN does not
    out, amax = orc.cast(3, 1, np.array([np.nan, -2.0, 1.0], np.float32), 3)
    assert amax == 2.0 and out.tolist() == [0x7FC0, 0xC000, 0x3F80]
    _, amax = orc.cast(3, 1, np.zeros(4, np.float32), 4, amax_in=-1.0)
    assert amax == -1.0  # a zero partial maximum is not committed
    _, amax = orc.cast(3, 1, np.array([0.5], np.float32), 1, amax_in=-1.0)
    assert amax == 0.5


# ---- quantize with the data's own amax (Float8Tensor.from_float) ----------------------------------
_TOP = {4: (57344.0, torch.float8_e5m2), 0: (448.0, torch.float8_e4m3fn)}


def _quant_inputs(rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * np.exp(rng.uniform(-8, 8, (rows, 1)))).astype(np.float32)
    x[1, :] = 0.0                                   # all-zero row: amax clamps to 1e-12
    x[2, 3] = np.inf                                # Inf row: scale 0, Inf * 0 = NaN
    x[3, 5] = np.nan                                # NaN row: NaN amax, NaN scale
    x[4, :] = rng.standard_normal(cols).astype(np.float32) * np.float32(1e-30)  # tiny: huge scale, saturation
    return x


def _reference_steps(x, fp8, per_row, margin):
    """tensor.py:60-74 (Float8Tensor.from_float) run with torch on the CPU; the per-tensor branch's
    e5ma_cast is the oracle's cast (pinned by the encoder tests above)."""
    import oracle
    top, tdt = _TOP[fp8]
    xf = torch.from_numpy(x)
    if per_row:
        amax = xf.abs().amax(dim=1).clamp_min(1e-12)
        scale = margin * top / amax
        data = (xf * scale[:, None]).clamp(-top, top).to(tdt).view(torch.uint8).numpy().reshape(-1)
        return data, (1.0 / scale).float().numpy(), xf.abs().amax(dim=1).numpy()
    amax = xf.abs().amax().clamp_min(1e-12).reshape(1)
    scale = (margin * top / amax).float()
    data, _ = oracle.cast(3, fp8, x.reshape(-1), x.size, 1.0, float(scale[0]))
    return data, (1.0 / scale).numpy(), xf.abs().amax().reshape(1).numpy()


def _same_f32(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a.view(np.uint32)[~np.isnan(a)],
                                                                      b.view(np.uint32)[~np.isnan(b)])


@pytest.mark.parametrize("fp8", [4, 0])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("margin", [1.0, 0.9])
def test_quantize_matches_reference_composition(orc, fp8, per_row, margin):
    """orc_quantize against the reference's own torch steps, bit for bit: codes, scale_inv, amax.  A NaN
    code from torch's .to(fp8) may carry the sign bit; the oracle's is 0x7F (the encoder's)."""
    rng = np.random.default_rng(7 + fp8 + per_row)
    rows, cols = 37, 203
    x = _quant_inputs(rng, rows, cols)
    top, _ = _TOP[fp8]
    qmax = float(np.float32(margin * top))
    got, sinv, amax = orc.quantize(3, fp8, x, rows, cols, qmax, per_row=per_row)
    want, want_sinv, want_amax = _reference_steps(x, fp8, per_row, margin)
    nan_code = (want & 0x7F) == 0x7F if fp8 == 0 else (want & 0x7F) > 0x7C
    assert np.all(got[nan_code] == 0x7F)
    assert np.array_equal(got[~nan_code], want[~nan_code])
    assert _same_f32(sinv, want_sinv) and _same_f32(amax, want_amax)


def test_quantize_special_cases(orc):
    """Closed forms: a tensor whose amax is a power of two maps it exactly to qmax; the all-zero tensor
    uses amax 1e-12; a NaN anywhere makes the per-tensor scale NaN; FP8 sources are decoded times sinv."""
    x = np.array([[0.25, -1.0, 0.5, 0.125]], np.float32)
    codes, sinv, amax = orc.quantize(3, 4, x, 1, 4, 57344.0)
    assert amax[0] == 1.0 and sinv[0] == np.float32(1.0) / np.float32(57344.0)
    assert codes.tolist() == [orc.encode(4, np.float32([14336.0]))[0], 0xFB, orc.encode(4, np.float32([28672.0]))[0],
                              orc.encode(4, np.float32([7168.0]))[0]]
    codes, sinv, amax = orc.quantize(3, 0, np.zeros((2, 8), np.float32), 2, 8, 448.0, per_row=True)
    r = np.float32(1.0) / np.float32(1e-12)
    assert np.all(codes == 0) and amax.tolist() == [0.0, 0.0]
    assert np.all(sinv == np.float32(1.0) / (r * np.float32(448.0)))
    codes, sinv, amax = orc.quantize(3, 4, np.array([1.0, np.nan, 2.0], np.float32), 1, 3, 57344.0)
    assert np.isnan(amax[0]) and np.isnan(sinv[0]) and np.all(codes == 0x7F)
    c8 = orc.encode(4, np.float32([3.0, -0.5, 0.75, 1.5]))
    got, s1, a1 = orc.quantize(4, 0, c8, 1, 4, 448.0, sinv=0.5)
    want, s2, a2 = orc.quantize(3, 0, orc.decode(4, c8, 0.5), 1, 4, 448.0)
    assert np.array_equal(got, want) and s1 == s2 and a1 == a2 == 1.5


# ---- GEMM semantics ----------------------------------------------------------------------------------
def _rand_fp8(rng, n, fmt):
    c = rng.integers(0, 256, n).astype(np.uint8)
    bad = (c & 0x7C) == 0x7C if fmt == 4 else (c & 0x7F) == 0x7F
    c[bad] ^= 4 if fmt == 4 else 1  # finite neighbours, as the reference fixtures draw them
    return c


def test_gemm_single_product_is_exact(orc):
    """With one non-zero k per output the FP32 sum is exact: D = convert((alpha*sa)*sb * a*b)."""
    rng = np.random.default_rng(1)
    m, n, k = 8, 8, 16
    A = np.zeros(k * m, np.uint8)
    B = np.zeros(k * n, np.uint8)
    a = _rand_fp8(rng, m, 4)
    b = _rand_fp8(rng, n, 0)
    A[np.arange(m) * k + 3] = a  # transa = T: A[kk + i*lda]
    B[np.arange(n) * k + 3] = b  # transb = N: B[kk + j*ldb]
    g = orc.Gemm(1, 0, m, n, k, 1.0, 4, A, k, 0, B, k, sa=[0.5], sb=[2.0], ddt=3)
    g.chain()
    va, vb = orc.decode(4, a).astype(np.float64), orc.decode(0, b).astype(np.float64)
    np.testing.assert_array_equal(g.D.reshape(n, m), np.outer(vb, va).astype(np.float32))


def _mk_case(orc, rng, ta, tb, at, bt, m, n, k):
    lda = (k if ta else m) + 16
    ldb = (k if not tb else n) + 16
    na, nb = lda * (m if ta else k), ldb * (n if not tb else k)
    def fill(dt, size):
        if dt in (4, 0):
            return _rand_fp8(rng, size, dt)
        x = rng.uniform(-2, 2, size).astype(np.float32)
        return orc.encode(dt, x) if dt == 1 else x
    return fill(at, na), lda, fill(bt, nb), ldb


@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("at,bt", [(4, 4), (4, 0), (0, 1), (3, 4), (1, 3)])
def test_gemm_chain_within_exact_bound(orc, ta, tb, at, bt):
    rng = np.random.default_rng(ta * 2 + tb)
    m, n, k = 37, 29, 48
    A, lda, B, ldb = _mk_case(orc, rng, ta, tb, at, bt, m, n, k)
    bias = rng.uniform(-8, 8, m).astype(np.float32)
    C = rng.uniform(-4, 4, (m + 1) * n).astype(np.float32)
    g = orc.Gemm(ta, tb, m, n, k, 1.25, at, A, lda, bt, B, ldb, sa=[0.37], sb=[1.9], beta=0.5, cdt=3, C=C, ldc=m + 1,
                 ddt=3, bias=bias, biasdt=3)
    amax = g.chain()
    iis, jjs = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    # the FFMA chain's own error is far inside the bound the kernels are held to
    bad, first, alo, ahi = g.check(g.D, C, iis.ravel(), jjs.ravel(), err_factor=1.0)
    assert bad == 0, first
    assert alo <= amax <= ahi


def test_gemm_check_rejects_planted_errors(orc):
    """Negative controls: a transposed operand, a dropped k term and a result off by a few ulps beyond
    the bound are all caught."""
    rng = np.random.default_rng(9)
    m, n, k = 32, 32, 64
    A, lda, B, ldb = _mk_case(orc, rng, 1, 0, 4, 4, m, n, k)
    iis, jjs = [a.ravel() for a in np.meshgrid(np.arange(m), np.arange(n), indexing="ij")]
    good = orc.Gemm(1, 0, m, n, k, 1.0, 4, A, lda, 4, B, ldb, ddt=3)
    good.chain()
    # 1. transposed operand: run the chain with transa flipped on the same bytes
    wrong = orc.Gemm(0, 0, m, n, k, 1.0, 4, A, lda, 4, B, ldb, ddt=3)
    wrong.chain()
    assert good.check(wrong.D, None, iis, jjs)[0] > m * n // 2
    # 2. a dropped term: zero one k column of A
    A2 = A.copy()
    A2[np.arange(m) * lda + 5] = 0
    dropped = orc.Gemm(1, 0, m, n, k, 1.0, 4, A2, lda, 4, B, ldb, ddt=3)
    dropped.chain()
    assert good.check(dropped.D, None, iis, jjs)[0] > 0
    # 3. one output moved by 2 * (bound + ulp)
    D = good.D.copy()
    ex, mag = good.exact(iis[:1], jjs[:1])
    D[0] = np.float32(ex[0] + 2 * (2 * k * mag[0] * 2.0 ** -24) + abs(ex[0]) * 2.0 ** -22 + 1e-30)
    assert good.check(D, None, iis, jjs)[0] == 1
    # 4. the sign of alpha flipped
    neg = orc.Gemm(1, 0, m, n, k, -1.0, 4, A, lda, 4, B, ldb, ddt=3)
    neg.chain()
    assert good.check(neg.D, None, iis, jjs)[0] > m * n // 2


def test_gemm_fp8_output_and_accumulate(orc):
    rng = np.random.default_rng(4)
    m, n, k = 20, 12, 32
    A, lda, B, ldb = _mk_case(orc, rng, 1, 0, 4, 0, m, n, k)
    D0 = rng.uniform(-1, 1, m * n).astype(np.float32)
    g = orc.Gemm(1, 0, m, n, k, 1.0, 4, A, lda, 0, B, ldb, beta=1.0, C=None, ddt=3, D=D0.copy(), ldd=m)
    g.chain()
    iis, jjs = [a.ravel() for a in np.meshgrid(np.arange(m), np.arange(n), indexing="ij")]
    ex, _ = g.exact(iis, jjs)
    np.testing.assert_allclose(g.D[jjs * m + iis], ex + D0[jjs * m + iis], rtol=1e-5, atol=1e-6)
    q = orc.Gemm(1, 0, m, n, k, 1.0, 4, A, lda, 0, B, ldb, ddt=4, qscale=0.25)
    amax = q.chain()
    f32 = orc.Gemm(1, 0, m, n, k, 1.0, 4, A, lda, 0, B, ldb, ddt=3)
    f32.chain()
    assert np.array_equal(q.D, orc.encode(4, f32.D, 0.25))
    assert amax == np.abs(f32.D).max()


# ---- Adam -------------------------------------------------------------------------------------------
def test_adam_closed_form_unit_moments(orc):
    """beta1 = beta2 = 0, eps = 0, no bias correction, no decay: m = g, v = RN(g*g), and
    u = g / sqrt(RN(g^2)) = +-1 exactly, so p_new = RN(p -+ lr)."""
    rng = np.random.default_rng(2)
    n = 10000
    p = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n).astype(np.float32) + np.float32(0.01))
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    cfg = dict(lr=1e-3, beta1=0.0, beta2=0.0, eps=0.0, weight_decay=0.0, step=1, adamw=1, bias_correction=0,
               grad_scale=1.0)
    p0 = p.copy()
    orc.adam(cfg, 3, p, 3, g, 3, m, v)
    assert np.array_equal(m, g) and np.array_equal(v, g * g)
    assert np.array_equal(p, p0 - np.sign(g).astype(np.float32) * np.float32(1e-3))


@pytest.mark.parametrize("adamw", [1, 0])
def test_adam_vs_torch_fp32(orc, adamw):
    rng = np.random.default_rng(8)
    n = 4096
    p = rng.standard_normal(n).astype(np.float32)
    tp = torch.nn.Parameter(torch.from_numpy(p.copy()))
    opt = (torch.optim.AdamW if adamw else torch.optim.Adam)([tp], lr=1e-2, weight_decay=0.1, foreach=False)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32)
        tp.grad = torch.from_numpy(g.copy())
        opt.step()
        cfg = dict(lr=1e-2, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1, step=step, adamw=adamw,
                   bias_correction=1, grad_scale=1.0)
        orc.adam(cfg, 3, p, 3, g, 3, m, v)
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-6, atol=1e-6)


def test_adam_fp8_copy_and_amax(orc):
    rng = np.random.default_rng(6)
    n = 1000
    p = orc.encode(1, rng.standard_normal(n).astype(np.float32))
    g = orc.encode(2, rng.standard_normal(n).astype(np.float32) * np.float32(0.1))
    m = orc.encode(1, rng.standard_normal(n).astype(np.float32) * np.float32(0.01))
    v = orc.encode(1, np.abs(rng.standard_normal(n)).astype(np.float32) * np.float32(1e-4))
    q = np.zeros(n, np.uint8)
    cfg = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=3, adamw=1, bias_correction=1,
               grad_scale=0.5)
    amax = orc.adam(cfg, 1, p, 2, g, 1, m, v, qdt=0, q=q, qscale=64.0)
    pf = orc.decode(1, p)
    # amax is max |p| of the FP32 values, before their BF16 rounding
    assert abs(amax - np.abs(pf).max()) <= np.abs(pf).max() * 2.0 ** -8 and amax != np.abs(pf).max()
    # the copy is taken from the FP32 value before its BF16 rounding: it agrees with the stored BF16
    # value to within one E4M3 rounding step
    ref = orc.encode(0, pf, 64.0)
    assert (np.abs(orc.decode(0, q).astype(np.float64) - orc.decode(0, ref)) <=
            np.abs(orc.decode(0, ref)) * 2.0 ** -3 + 2.0 ** -9).all()


# ---- Adam's operation order, bit for bit -------------------------------------------------------------
def _rn32(x):
    """Round a Fraction to the nearest float32 (ties to even), exactly; overflow to +-inf."""
    from fractions import Fraction
    if x == 0:
        return np.float32(0.0)
    sign, x = (-1 if x < 0 else 1), abs(Fraction(x))
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    e = max(e, -126)                  # below 2^-126 the grid is the subnormal one, spacing 2^-149
    q = x / Fraction(2) ** (e - 23)   # the significand on a 24-bit integer grid
    n, r = divmod(q.numerator, q.denominator)
    if 2 * r > q.denominator or (2 * r == q.denominator and n % 2 == 1):
        n += 1
    v = float(n) * 2.0 ** (e - 23)
    return np.float32(sign * v) if abs(v) < 2.0 ** 128 else np.float32(sign * np.inf)


def _adam_exact_model(cfg, p, g, m, v):
    """One step of include/e5m2effma.h's documented order on float32 values, each operation rounded once
    from its exact value (an FMA: one rounding of a * b + c).  Coefficients as the host forms them: in
    double, rounded to float32 once (reference src/adamw_e5m2effma.cu:150-157)."""
    from fractions import Fraction as Fr
    import math
    f = lambda x: Fr(float(x))
    c1, c2 = np.float32(1.0 - float(np.float32(cfg["beta1"]))), np.float32(1.0 - float(np.float32(cfg["beta2"])))
    b1, b2 = np.float32(cfg["beta1"]), np.float32(cfg["beta2"])
    corr = lambda b: np.float32(1.0 / (1.0 - float(b) ** cfg["step"])) if cfg["bias_correction"] else np.float32(1)
    r1, r2 = corr(b1), corr(b2)
    lr, wd, eps = np.float32(cfg["lr"]), np.float32(cfg["weight_decay"]), np.float32(cfg["eps"])
    decay = np.float32(float(lr) * float(wd))
    gs = np.float32(cfg["grad_scale"] or 1.0)
    out = []
    for pi, gi, mi, vi in zip(p, g, m, v):
        gg = _rn32(f(gi) * f(gs))
        if not cfg["adamw"]:
            gg = _rn32(f(wd) * f(pi) + f(gg))
        mm = _rn32(f(b1) * f(mi) + f(_rn32(f(c1) * f(gg))))
        vv = _rn32(f(b2) * f(vi) + f(_rn32(f(c2) * f(_rn32(f(gg) * f(gg))))))
        num = _rn32(f(mm) * f(r1))
        root = np.float32(math.sqrt(float(_rn32(f(vv) * f(r2)))))  # 53 >= 2 * 24 + 2: double rounding is exact
        u = _rn32(f(num) / f(_rn32(f(root) + f(eps))))
        pp = pi
        if cfg["adamw"]:
            pp = _rn32(-f(decay) * f(pp) + f(pp))
        pp = _rn32(-f(lr) * f(u) + f(pp))
        out.append((pp, mm, vv))
    return [np.array(c, np.float32) for c in zip(*out)]


@pytest.mark.parametrize("adamw,bc", [(1, 1), (0, 1), (1, 0)])
def test_adam_order_matches_exact_model(orc, adamw, bc):
    """The oracle's Adam step, bit for bit, against the exact-arithmetic model of the documented order on
    random state over several steps.  A misplaced or missing FMA (m, v, the weight decay) changes the
    result in a sizeable fraction of these elements."""
    rng = np.random.default_rng(40 + adamw + 2 * bc)
    n = 1500
    p = (rng.standard_normal(n) * 0.5).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    v = (np.abs(rng.standard_normal(n)) * 1e-4).astype(np.float32)
    for step in (1, 2, 7):
        g = (rng.standard_normal(n) * 3e-2).astype(np.float32)
        cfg = dict(lr=3e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.05, step=step, adamw=adamw,
                   bias_correction=bc, grad_scale=0.75)
        want_p, want_m, want_v = _adam_exact_model(cfg, p, g, m, v)
        orc.adam(cfg, 3, p, 3, g, 3, m, v)
        assert np.array_equal(p.view(np.uint32), want_p.view(np.uint32)), step
        assert np.array_equal(m.view(np.uint32), want_m.view(np.uint32)), step
        assert np.array_equal(v.view(np.uint32), want_v.view(np.uint32)), step


def test_adam_exact_model_detects_a_misplaced_fma(orc):
    """Negative control: the same model with m's update as two roundings (mul, then add) disagrees with
    the oracle on these inputs, so the comparison above can tell the orders apart."""
    from fractions import Fraction as Fr
    rng = np.random.default_rng(47)
    n = 1500
    p = (rng.standard_normal(n) * 0.5).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    v = (np.abs(rng.standard_normal(n)) * 1e-4).astype(np.float32)
    g = (rng.standard_normal(n) * 3e-2).astype(np.float32)
    b1, c1 = np.float32(0.9), np.float32(1.0 - float(np.float32(0.9)))
    fused = [_rn32(Fr(float(b1)) * Fr(float(mi)) + Fr(float(_rn32(Fr(float(c1)) * Fr(float(gi))))))
             for mi, gi in zip(m, g)]
    split = [np.float32(b1 * mi) + _rn32(Fr(float(c1)) * Fr(float(gi))) for mi, gi in zip(m, g)]
    assert sum(a != b for a, b in zip(fused, split)) > n // 20
    cfg = dict(lr=3e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.05, step=1, adamw=1,
               bias_correction=1, grad_scale=1.0)
    orc.adam(cfg, 3, p, 3, g, 3, m, v)
    assert np.array_equal(m, np.array(fused, np.float32)) and not np.array_equal(m, np.array(split, np.float32))


# ---- BASELINE config 1's CPU path: the reference's MAC chain --------------------------------------------
def test_lane_gemm_matches_reference_lane_and_closed_form(orc):
    rng = np.random.default_rng(51)
    M, N, K = 24, 20, 48
    a = orc.encode(4, (rng.standard_normal(M * K) * 4).astype(np.float32))
    b = orc.encode(4, (rng.standard_normal(K * N) * 4).astype(np.float32))
    got = orc.lane_gemm(a, b, M, N, K, 1, 1, threads=3)
    ref = orc.ref_library()
    if ref is not None:
        assert np.array_equal(got, orc.lane_gemm(a, b, M, N, K, 1, 1, fn=ref.ref_lane))
    # one non-zero product per output: the chain is BF16 of that product (+0 start, one rounding)
    a1 = np.zeros(M * K, np.uint8)
    b1 = np.zeros(K * N, np.uint8)
    a1[np.arange(M) * K + 5] = a[:M]
    b1[5 * N + np.arange(N)] = b[:N]
    one = orc.lane_gemm(a1, b1, M, N, K, 1, 1)
    prod = np.outer(orc.decode(4, a[:M]).astype(np.float64), orc.decode(4, b[:N]).astype(np.float64))
    assert np.array_equal(one, orc.encode(1, prod.astype(np.float32)).reshape(M, N))


@pytest.mark.parametrize("n", [1, 8, 40])
def test_chain_is_independent_of_the_thread_split(orc, n):
    """The CPU chain splits columns, or rows for a GEMV; every output's chain is the same either way."""
    rng = np.random.default_rng(60 + n)
    M, K = 96, 256
    a = orc.encode(orc.E5M2, (rng.standard_normal(M * K) * 2).astype(np.float32))
    b = orc.encode(orc.BF16, rng.standard_normal(K * n).astype(np.float32))
    outs = []
    for th in (1, 5):
        g = orc.Gemm(1, 0, M, n, K, 1.0, orc.E5M2, a, K, orc.BF16, b, K, ddt=orc.FP32)
        g.chain(threads=th)
        outs.append(g.D.copy())
    assert np.array_equal(outs[0], outs[1])
