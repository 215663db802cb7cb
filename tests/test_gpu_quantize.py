"""e5ma_quantize on the GPU through the C ABI, bit-exact against the oracle (which restates the reference's
Float8Tensor.from_float steps, binds/python/e5m2effma/tensor.py:60-74): codes, scale_inv and amax, per
tensor and per row, every source dtype, both FP8 formats, NaN / Inf / all-zero groups, ragged and
unaligned shapes (the scalar and re-reading kernels as well as the register-resident one), and the
reference's own torch composition run on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
import e5m2effma_amd as fx
from e5m2effma_amd import _lib

pytestmark = pytest.mark.gpu
TOP = {oracle.E5M2: 57344.0, oracle.E4M3: 448.0}


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def gpu_quantize(dev, tin, tout, x, rows, cols, qmax, per_row, sinv=None, offset_in=0, offset_out=0):
    """e5ma_quantize of numpy array x (codes of tin); returns (codes, scale_inv, amax)."""
    keep = []
    xt, px = gu.to_dev(np.ascontiguousarray(x, gu.NPD[tin]), dev, offset_in)
    n = rows * cols
    out = torch.empty(n + offset_out + 16, dtype=torch.uint8, device=dev)
    po = out.data_ptr() + offset_out
    g = rows if per_row else 1
    sc = torch.full((g,), -7.0, dtype=torch.float32, device=dev)  # garbage: the call must write every entry
    am = torch.full((g,), -7.0, dtype=torch.float32, device=dev)
    sp = None
    if sinv is not None:
        t, sp = gu.dev_floats(sinv, dev)
        keep.append(t)
    S = _lib.tensor(px, tin, sp)
    D = _lib.tensor(po, tout, scaling=_lib.SCALING_OUTER if per_row else _lib.SCALING_TENSOR)
    s = _lib.lib().e5ma_quantize(ctypes.byref(S), ctypes.byref(D), rows, cols, qmax, sc.data_ptr(), am.data_ptr(),
                                 ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert s == 0, (s, _lib.last_error())
    torch.cuda.synchronize(dev)
    return gu.from_dev(out, po, np.uint8, n), sc.cpu().numpy(), am.cpu().numpy()


def same_f32(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])


def source(rng, tin, rows, cols):
    x = (rng.standard_normal((rows, cols)) * np.exp(rng.uniform(-6, 6, (rows, 1)))).astype(np.float32)
    if rows > 4:
        x[1, :] = 0.0
        x[2, cols // 2] = np.inf
        x[3, cols - 1] = np.nan
    if tin == oracle.FP32:
        return x.reshape(-1)
    if tin in gu.FP8:
        return oracle.encode(tin, x.reshape(-1), 1.0 / max(1e-30, float(np.nanmax(np.abs(x[np.isfinite(x)])))) * 100)
    return oracle.encode(tin, x.reshape(-1))


@pytest.mark.parametrize("tin", [oracle.FP32, oracle.BF16, oracle.FP16, oracle.E5M2, oracle.E4M3])
@pytest.mark.parametrize("tout", [oracle.E5M2, oracle.E4M3])
@pytest.mark.parametrize("per_row", [False, True])
def test_quantize_dtypes_bit_exact(dev, tin, tout, per_row):
    rng = np.random.default_rng(10 * tin + tout + per_row)
    rows, cols = 67, 1024 + 48
    x = source(rng, tin, rows, cols)
    sinv = 0.375 if tin in gu.FP8 else None
    qmax = TOP[tout]
    got = gpu_quantize(dev, tin, tout, x, rows, cols, qmax, per_row, sinv=sinv)
    want = oracle.quantize(tin, tout, x, rows, cols, qmax, per_row=per_row, sinv=sinv or 1.0)
    assert np.array_equal(got[0], want[0])
    assert same_f32(got[1], want[1]) and same_f32(got[2], want[2])


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 17), (5, 16), (9, 8192), (4, 8192 + 16), (130, 4096), (2, 100003),
                                       (1, 1 << 20)])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("off", [(0, 0), (4, 1)])
def test_quantize_shapes_and_alignment(dev, rows, cols, per_row, off):
    """every kernel variant: register-resident rows (cols % 16 == 0, <= 8192), re-read rows (longer), the
    element-wise paths (ragged or unaligned), and per-tensor grids from one element to many blocks"""
    rng = np.random.default_rng(rows * 7 + cols + off[0])
    x = (rng.standard_normal(rows * cols) * 3).astype(np.float32)
    got = gpu_quantize(dev, oracle.FP32, oracle.E4M3, x, rows, cols, 0.9 * 448.0, per_row, offset_in=off[0],
                       offset_out=off[1])
    want = oracle.quantize(oracle.FP32, oracle.E4M3, x, rows, cols, np.float32(0.9 * 448.0), per_row=per_row)
    assert np.array_equal(got[0], want[0])
    assert same_f32(got[1], want[1]) and same_f32(got[2], want[2])


def test_quantize_special_groups(dev):
    """a NaN makes its group's amax and scale NaN and every code 0x7F; an Inf gives scale 0; an all-zero
    group maps amax 1e-12; calls in a row do not see the previous call's reduction word"""
    rows, cols = 6, 64
    x = np.ones((rows, cols), np.float32)
    x[0, 5] = np.nan
    x[1, 7] = -np.inf
    x[2, :] = 0.0
    x = x.reshape(-1)
    for per_row in (True, False):
        got = gpu_quantize(dev, oracle.FP32, oracle.E5M2, x, rows, cols, 57344.0, per_row)
        want = oracle.quantize(oracle.FP32, oracle.E5M2, x, rows, cols, 57344.0, per_row=per_row)
        assert np.array_equal(got[0], want[0]) and same_f32(got[1], want[1]) and same_f32(got[2], want[2])
    assert np.isnan(got[2][0]) and np.all(got[0] == 0x7F)
    y = np.full(4096, 2.0, np.float32)
    got = gpu_quantize(dev, oracle.FP32, oracle.E5M2, y, 1, 4096, 57344.0, False)
    assert got[2][0] == 2.0 and got[1][0] == np.float32(1.0) / (np.float32(0.5) * np.float32(57344.0))
    assert np.all(got[0] == 0x7B)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("fp8", [torch.float8_e5m2, torch.float8_e4m3fn])
def test_quantize_matches_reference_steps_on_gpu(dev, per_row, fp8):
    """fx.quantize against the reference's Float8Tensor.from_float steps (tensor.py:64-74) executed with
    torch on the GPU (per tensor: torch amax / reciprocal, then e5ma_cast)"""
    g = torch.Generator(device="cpu").manual_seed(3)
    x = (torch.randn(300, 2048, generator=g) * torch.logspace(-3, 3, 300)[:, None]).to(dev)
    top = 57344.0 if fp8 == torch.float8_e5m2 else 448.0
    codes, sinv, amax = fx.quantize(x, fp8, per_row=per_row, margin=0.9)
    if per_row:
        a = x.abs().amax(dim=1).clamp_min(1e-12)
        scale = 0.9 * top / a
        want = (x * scale[:, None]).clamp(-top, top).to(fp8)
    else:
        a = x.abs().amax().clamp_min(1e-12).reshape(1)
        scale = (0.9 * top / a).float()
        want = fx.cast(x, fp8, scale=scale)
    assert torch.equal(codes.view(torch.uint8), want.view(torch.uint8))
    assert torch.equal(sinv, (1.0 / scale).float().reshape(-1))
    assert torch.equal(amax, x.abs().amax(dim=1) if per_row else x.abs().amax().reshape(1))


def test_from_float_uses_quantize(dev):
    w = torch.randn(96, 160, device=dev) * 0.02
    for per_row in (False, True):
        t = fx.Float8Tensor.from_float(w, fp8=torch.float8_e4m3fn, per_row=per_row)
        codes, sinv, _ = fx.quantize(w, torch.float8_e4m3fn, per_row=per_row)
        assert torch.equal(t._data.view(torch.uint8), codes.view(torch.uint8)) and torch.equal(t._scale_inv, sinv)
