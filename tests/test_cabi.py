"""The C ABI without a GPU: the library loads, exports every function include/e5m2effma.h declares,
has the reference's struct layouts, and rejects bad arguments with the reference's status codes and
messages before touching a device (reference src/gemm_e5m2effma.cu:55-81, src/e5m2effma.cu:88-95,
src/adamw_e5m2effma.cu:131-147)."""
import ctypes
import os
import re

import pytest

from e5m2effma_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E4M3, BF16, FP16, FP32, E5M2 = 0, 1, 2, 3, 4
FAKE = 0x10000  # a non-NULL, 16-byte aligned address that is never dereferenced (validation fails first)


def header_functions():
    names = set()
    for h in ("e5m2effma.h", "e5m2effma_ext.h"):
        with open(os.path.join(ROOT, "include", h)) as f:
            text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
        names |= set(re.findall(r"\b(e5ma_\w+)\s*\(", text))
    return sorted(names)


def test_exports_every_declared_function():
    names = header_functions()
    assert set(names) == set(_lib.EXPORTS)
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n


def test_struct_layouts_match_reference():
    # reference include/e5m2effma.h:61-70, 95-101 on LP64
    assert ctypes.sizeof(_lib.Tensor) == 48
    assert _lib.Tensor.scaling.offset == 40
    assert ctypes.sizeof(_lib.AdamConfig) == 36


def test_status_strings():
    assert [_lib.status_string(s) for s in range(4)] == ["E5MA_OK", "E5MA_INVALID_VALUE", "E5MA_NOT_SUPPORTED",
                                                        "E5MA_CUDA_ERROR"]
    assert _lib.status_string(17) == "unknown e5ma_status"


def T(dtype=E5M2, data=FAKE, scaling=0, scale_inv=None):
    return _lib.tensor(data, dtype, scale_inv, None, None, scaling)


def gemm(transa=1, transb=0, m=32, n=32, k=32, A=None, lda=32, B=None, ldb=32, beta=0.0, C=None, ldc=32, D=None,
         ldd=32, bias=None, alpha=1.0):
    A = T() if A is None else A
    B = T() if B is None else B
    D = T(BF16) if D is None else D
    L = _lib.lib()
    return L.e5ma_gemm(transa, transb, m, n, k, alpha, _lib.ref(A), lda, _lib.ref(B), ldb, beta, _lib.ref(C), ldc,
                       _lib.ref(D), ldd, _lib.ref(bias), None), _lib.last_error()


GEMM_ERRORS = [
    (dict(A=T(data=None)), 1, "e5ma_gemm: A, B, D or their data is NULL"),
    (dict(transa=2), 1, "e5ma_gemm: transa / transb must be E5MA_OP_N or E5MA_OP_T"),
    (dict(m=-1), 1, "e5ma_gemm: negative size (m=-1 n=32 k=32)"),
    (dict(D=T(7)), 1, "e5ma_gemm: invalid D dtype 7"),
    (dict(A=T(FP16)), 2, "e5ma_gemm: A and B must be E5M2, E4M3, BF16 or FP32 (got dtypes 2, 4)"),
    (dict(k=24), 1, "e5ma_gemm: k = 24 is not a multiple of 16"),
    (dict(lda=40), 1, "e5ma_gemm: lda = 40 / ldb = 32 must be multiples of 16"),
    (dict(A=T(data=FAKE + 8)), 1, "e5ma_gemm: A and B must be 16-byte aligned"),
    (dict(k=48, lda=32), 1, "e5ma_gemm: lda = 32 < 48"),
    (dict(transb=1, n=48, ldb=32), 1, "e5ma_gemm: ldb = 32 < 48"),
    (dict(ldd=16), 1, "e5ma_gemm: ldd = 16 < m = 32"),
    (dict(bias=T(9)), 1, "e5ma_gemm: invalid bias dtype 9"),
    (dict(beta=1.0, C=T(9)), 1, "e5ma_gemm: invalid C dtype 9"),
    (dict(beta=1.0, C=T(FP32), ldc=16), 1, "e5ma_gemm: ldc = 16 < m = 32"),
    (dict(A=T(scaling=3)), 1, "e5ma_gemm: invalid scaling of A or B"),
    (dict(A=T(scaling=1)), 1, "e5ma_gemm: E5MA_SCALING_OUTER needs an FP8 operand with a scale_inv vector"),
    (dict(B=T(BF16, scaling=1, scale_inv=FAKE)), 1,
     "e5ma_gemm: E5MA_SCALING_OUTER needs an FP8 operand with a scale_inv vector"),
    (dict(D=T(BF16, scaling=1)), 1, "e5ma_gemm: C, D and bias take per-tensor scaling only"),
]


@pytest.mark.parametrize("kw,status,msg", GEMM_ERRORS)
def test_gemm_validation(kw, status, msg):
    s, err = gemm(**kw)
    assert (s, err) == (status, msg)


def test_gemm_zero_sizes_return_ok_before_device():
    assert gemm(m=0) == (0, "")
    assert gemm(n=0, k=24) == (0, "")  # zero sizes return before the k check, as the reference does


def test_error_cleared_by_next_call():
    assert gemm(k=24)[0] == 1
    assert gemm(m=0) == (0, "")


def test_cast_validation():
    L = _lib.lib()
    c = lambda s, d, n=16: (L.e5ma_cast(_lib.ref(s), _lib.ref(d), n, None), _lib.last_error())
    assert c(T(FP32, data=None), T(E5M2)) == (1, "e5ma_cast: src / dst or their data is NULL")
    assert c(T(FP32), T(5)) == (1, "e5ma_cast: invalid dtype (src 3, dst 5)")
    assert c(T(FP32), T(E5M2, scaling=1)) == (1, "e5ma_cast: per-tensor scaling only")
    assert c(T(FP32), T(E5M2), 0) == (0, "")


def test_quantize_validation():
    """e5ma_quantize (include/e5m2effma_ext.h) rejects bad arguments before any device call"""
    L = _lib.lib()
    q = lambda s, d, rows=4, cols=16, qmax=448.0, sc=FAKE: (
        L.e5ma_quantize(_lib.ref(s), _lib.ref(d), rows, cols, qmax, sc, None, None), _lib.last_error())
    assert q(T(FP32, data=None), T(E4M3)) == (1, "e5ma_quantize: src / dst, their data or scale_inv is NULL")
    assert q(T(FP32), T(E4M3), sc=None)[0] == 1
    assert q(T(FP32), T(BF16)) == (1, "e5ma_quantize: src dtype 3 / dst dtype 1 (dst must be E5MA_E4M3 or E5MA_E5M2)")
    assert q(T(FP32, scaling=1), T(E4M3)) == (1, "e5ma_quantize: src takes per-tensor scaling only")
    assert q(T(FP32), T(E4M3, scaling=2)) == (1, "e5ma_quantize: invalid dst scaling 2")
    assert q(T(FP32), T(E5M2), qmax=0.0) == (1, "e5ma_quantize: qmax = 0 must be positive and finite")
    assert q(T(FP32), T(E5M2), qmax=float("inf"))[0] == 1
    assert q(T(FP32), T(E5M2), qmax=float("nan"))[0] == 1
    assert q(T(FP32), T(E5M2, scaling=1), rows=0) == (0, "")
    assert q(T(FP32), T(E5M2), cols=0) == (0, "")
    assert q(T(FP32), T(E5M2), rows=1 << 40, cols=1 << 40) == (1, "e5ma_quantize: rows x cols overflows")
    assert q(T(FP32), T(E5M2, scaling=1), rows=1 << 24, cols=16) == (
        1, "e5ma_quantize: per-row scaling takes at most 16777215 rows, got 16777216")


def test_adam_validation():
    L = _lib.lib()
    cfg = _lib.AdamConfig(1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 1, 1, 1.0)

    def a(p=None, g=None, m=None, v=None, q=None, n=16, c=cfg):
        p = T(FP32) if p is None else p
        g = T(FP32) if g is None else g
        m = T(FP32) if m is None else m
        v = T(FP32) if v is None else v
        s = L.e5ma_adam(ctypes.byref(c) if c is not None else None, n, _lib.ref(p), _lib.ref(g), _lib.ref(m),
                        _lib.ref(v), _lib.ref(q), None)
        return s, _lib.last_error()
    assert a(c=None)[0] == 1
    assert a(g=T(FP32, data=None)) == (1, "e5ma_adam: cfg, param, grad, exp_avg, exp_avg_sq or their data is NULL")
    bad_step = _lib.AdamConfig(1e-3, 0.9, 0.999, 1e-8, 0.0, 0, 1, 1, 1.0)
    assert a(c=bad_step) == (1, "e5ma_adam: step = 0, must be >= 1")
    assert a(p=T(FP16)) == (2, "e5ma_adam: param must be FP32 or BF16 (dtype 2)")
    assert a(v=T(BF16)) == (2, "e5ma_adam: exp_avg and exp_avg_sq must both be FP32 or both BF16 (dtypes 3, 1)")
    assert a(g=T(E5M2)) == (2, "e5ma_adam: grad must be FP32, BF16 or FP16 (dtype 4)")
    assert a(q=T(BF16)) == (1, "e5ma_adam: param_fp8 must have dtype E5MA_E4M3 or E5MA_E5M2 (dtype 1)")
    assert a(q=T(E5M2, scaling=1)) == (1, "e5ma_adam: param_fp8 takes per-tensor scaling only")
    assert a(n=0) == (0, "")


def test_no_device_is_a_runtime_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    s, err = gemm()
    assert s == 3 and err.startswith("hipGetDevice: HIP error")


def test_gemm_ex_and_workspace_query_validation():
    """e5ma_gemm_ex checks its workspace first, then runs e5ma_gemm's rules with its own name;
    e5ma_gemm_workspace_size checks its arguments before any device use."""
    L = _lib.lib()
    A, B, D = T(), T(), T(BF16)
    ex = lambda ws, nbytes, k=32: (L.e5ma_gemm_ex(1, 0, 32, 32, k, 1.0, _lib.ref(A), 32, _lib.ref(B), 32, 0.0, None, 0,
                                                  _lib.ref(D), 32, None, ws, nbytes, None), _lib.last_error())
    assert ex(FAKE + 16, 4096) == (1, "e5ma_gemm_ex: a workspace of 4096 bytes needs a 256-byte aligned pointer")
    assert ex(None, 4096) == (1, "e5ma_gemm_ex: a workspace of 4096 bytes needs a 256-byte aligned pointer")
    assert ex(FAKE, 4096, k=24) == (1, "e5ma_gemm_ex: k = 24 is not a multiple of 16")
    assert ex(None, 0, k=24) == (1, "e5ma_gemm_ex: k = 24 is not a multiple of 16")
    out = ctypes.c_size_t(7)
    ws = lambda *a: (L.e5ma_gemm_workspace_size(*a), _lib.last_error())
    assert ws(1, 0, 32, 32, 32, E5M2, 32, E5M2, 32, None) == (1, "e5ma_gemm_workspace_size: bytes is NULL")
    assert ws(2, 0, 32, 32, 32, E5M2, 32, E5M2, 32, ctypes.byref(out))[0] == 1
    assert ws(1, 0, 32, 32, 32, FP16, 32, E5M2, 32, ctypes.byref(out))[0] == 2
    assert ws(1, 0, 0, 32, 32, E5M2, 32, E5M2, 32, ctypes.byref(out)) == (0, "") and out.value == 0
    assert ws(1, 0, 32, 4, 32, E5M2, 32, BF16, 32, ctypes.byref(out)) == (0, "") and out.value == 0  # GEMV route


def test_gemm_noalloc_validation():
    """e5ma_gemm_noalloc runs e5ma_gemm's rules, with its own name, before any device use."""
    L = _lib.lib()
    A, B, D = T(), T(), T(BF16)
    na = lambda k=32, m=32: (L.e5ma_gemm_noalloc(1, 0, m, 32, k, 1.0, _lib.ref(A), 32, _lib.ref(B), 32, 0.0, None, 0,
                                                 _lib.ref(D), 32, None, None), _lib.last_error())
    assert na(k=24) == (1, "e5ma_gemm_noalloc: k = 24 is not a multiple of 16")
    assert na(m=-1) == (1, "e5ma_gemm_noalloc: negative size (m=-1 n=32 k=32)")
    assert na(m=0) == (0, "")
