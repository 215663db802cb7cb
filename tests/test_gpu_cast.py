"""e5ma_cast on the GPU, bit-exact against the oracle (reference src/e5m2effma.cu:53-63): every dtype
pair over every FP8 / 16-bit code and random FP32 bit patterns, tails and unaligned buffers, amax, and
the FP32 -> E5M2 / E4M3 / BF16 encoders over all 2^32 inputs."""
import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
DTYPES = [oracle.E4M3, oracle.BF16, oracle.FP16, oracle.FP32, oracle.E5M2]


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def source_values(rng, tin):
    if tin in (oracle.E4M3, oracle.E5M2):
        return np.concatenate([np.arange(256, dtype=np.uint8), rng.integers(0, 256, 5000).astype(np.uint8)])
    if tin in (oracle.BF16, oracle.FP16):
        return np.concatenate([np.arange(65536, dtype=np.uint32).astype(np.uint16),
                               rng.integers(0, 65536, 5000).astype(np.uint16)])
    u = rng.integers(0, 1 << 32, 300000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x47600000, 0x47700000, 0x43E00000,
                        0x43F00000, 0x00000001, 0x37800000, 0x3B000000], np.uint32)
    return np.concatenate([u, special]).view(np.float32)


def same(got, want, tout):
    if tout in (oracle.FP32, oracle.FP16):  # NaN payloads are not part of the contract; all other bits are
        g, w = oracle.decode(tout, got), oracle.decode(tout, want)
        bits = np.uint32 if tout == oracle.FP32 else np.uint16
        ok = ~np.isnan(w)
        return np.array_equal(np.isnan(g), np.isnan(w)) and np.array_equal(got[ok].view(bits), want[ok].view(bits))
    return np.array_equal(got, want)


@pytest.mark.parametrize("tin", DTYPES)
@pytest.mark.parametrize("tout", DTYPES)
def test_cast_pairs_bit_exact(dev, tin, tout):
    rng = np.random.default_rng(tin * 8 + tout)
    x = source_values(rng, tin)
    fp8_in, fp8_out = tin in gu.FP8, tout in gu.FP8
    sinv = 0.75 if fp8_in else None
    qs = 0.5 if fp8_out else None
    got, amax = gu.gpu_cast(dev, tin, tout, x, sinv=sinv, qscale=qs)
    want, want_amax = oracle.cast(tin, tout, x, x.size, sinv or 1.0, qs or 1.0, 0.0)
    assert same(got, want, tout)
    assert np.float32(amax).view(np.uint32) == np.float32(want_amax).view(np.uint32)


@pytest.mark.parametrize("n", [1, 15, 16, 17, 4099, 100003])
@pytest.mark.parametrize("off_in,off_out", [(0, 0), (1, 3), (4, 0), (0, 2)])
def test_cast_tails_and_alignment(dev, n, off_in, off_out):
    rng = np.random.default_rng(n + off_in)
    x = (rng.standard_normal(n) * 1000).astype(np.float32)
    x[rng.integers(0, n, max(1, n // 500))] = np.float32(np.nan)
    got, amax = gu.gpu_cast(dev, oracle.FP32, oracle.E4M3, x, qscale=0.25, offset_in=4 * off_in, offset_out=off_out)
    want, want_amax = oracle.cast(oracle.FP32, oracle.E4M3, x, n, 1.0, 0.25, 0.0)
    assert np.array_equal(got, want) and np.float32(amax) == np.float32(want_amax)
    b16 = oracle.encode(oracle.BF16, x)
    got, amax = gu.gpu_cast(dev, oracle.BF16, oracle.E5M2, b16, offset_in=2 * off_in, offset_out=off_out)
    want, want_amax = oracle.cast(oracle.BF16, oracle.E5M2, b16, n, 1.0, 1.0, 0.0)
    assert np.array_equal(got, want) and np.float32(amax) == np.float32(want_amax)


def test_cast_amax_rules(dev):
    # NaN never enters amax, Inf does; a zero maximum is not committed; the value in *amax is max-reduced
    x = np.array([np.nan, -2.0, 1.0], np.float32)
    _, amax = gu.gpu_cast(dev, oracle.FP32, oracle.BF16, x)
    assert amax == 2.0
    _, amax = gu.gpu_cast(dev, oracle.FP32, oracle.BF16, np.zeros(70000, np.float32), amax0=-1.0)
    assert amax == -1.0
    _, amax = gu.gpu_cast(dev, oracle.FP32, oracle.BF16, np.full(70000, 0.5, np.float32), amax0=3.0)
    assert amax == 3.0
    codes, amax = gu.gpu_cast(dev, oracle.FP32, oracle.E5M2, np.array([1.0, np.inf, -1e6, 3.0], np.float32))
    assert codes.tolist() == [0x3C, 0x7B, 0xFB, 0x42] and amax == np.inf  # reference python KAT


def test_cast_config2_scale_from_amax(dev):
    """BASELINE config 2 cast leg at reduced size: amax pre-pass, scale = 57344 / amax (E5M2) or
    448 / amax (E4M3), quantize with that scale."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal(1 << 20) * 0.02).astype(np.float32)
    _, amax = gu.gpu_cast(dev, oracle.FP32, oracle.BF16, w)
    assert np.float32(amax) == np.abs(w).max()
    for fmt, top in ((oracle.E5M2, 57344.0), (oracle.E4M3, 448.0)):
        qs = np.float32(top) / np.float32(amax)
        got, a2 = gu.gpu_cast(dev, oracle.FP32, fmt, w, qscale=qs)
        want, _ = oracle.cast(oracle.FP32, fmt, w, w.size, 1.0, float(qs), 0.0)
        assert np.array_equal(got, want) and a2 == amax
        assert (got & 0x7F).max() == (0x7B if fmt == oracle.E5M2 else 0x7E)


def _cast_dev(src, tin, tout, out):
    import ctypes
    from e5m2effma_amd import _lib
    S, D = _lib.tensor(src.data_ptr(), tin), _lib.tensor(out.data_ptr(), tout)
    s = _lib.lib().e5ma_cast(ctypes.byref(S), ctypes.byref(D), src.numel(),
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert s == 0


@pytest.mark.parametrize("aligned", [True, False])
def test_encoders_exhaustive_2pow32(dev, aligned):
    """All 2^32 FP32 bit patterns -> E5M2, E4M3, BF16 on the GPU, against torch's conversions inside
    the finite range (both round to nearest even) and the satfinite / NaN rules outside it.  Aligned buffers
    take the 16-byte path (four FP8 codes per pair of conversion instructions); a destination one byte off
    takes the element path (one code per conversion)."""
    chunk = 1 << 27
    out8 = torch.empty(chunk + 16, dtype=torch.uint8, device=dev)[0 if aligned else 1:][:chunk]
    out16 = torch.empty(chunk, dtype=torch.int16, device=dev)
    for c in range((1 << 32) // chunk):
        bits = (torch.arange(chunk, dtype=torch.int64, device=dev) + c * chunk).to(torch.int32)
        x = bits.view(torch.float32)
        a = x.abs()
        nan = torch.isnan(x)
        neg = (bits < 0)
        for fmt, tdt, top, topcode in ((oracle.E5M2, torch.float8_e5m2, 57344.0, 0x7B),
                                       (oracle.E4M3, torch.float8_e4m3fn, 448.0, 0x7E)):
            _cast_dev(x, oracle.FP32, fmt, out8)
            inr = a < top
            ref = torch.where(inr, x.masked_fill(~inr, 0).to(tdt).view(torch.uint8),
                              torch.where(nan, torch.full_like(out8, 0x7F),
                                          (neg.to(torch.uint8) << 7) | topcode))
            assert torch.equal(out8, ref), f"E{fmt} chunk {c}"
        if aligned:
            _cast_dev(x, oracle.FP32, oracle.BF16, out16)
            ref16 = torch.where(nan, torch.full_like(out16, 0x7FC0),
                                x.masked_fill(nan, 0).to(torch.bfloat16).view(torch.int16))
            assert torch.equal(out16, ref16), f"BF16 chunk {c}"
