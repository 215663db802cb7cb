"""ctypes binding of the C ABI in ``include/e5m2effma.h`` and ``include/e5m2effma_ext.h``
(``libe5m2effma.so``, built in-tree).

Loading fails loudly when the library is missing: there is no fallback path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libe5m2effma.so")

E4M3, BF16, FP16, FP32, E5M2 = 0, 1, 2, 3, 4
OP_N, OP_T = 0, 1
OK, INVALID_VALUE, NOT_SUPPORTED, HIP_ERROR = 0, 1, 2, 3
SCALING_TENSOR, SCALING_OUTER = 0, 1

# every symbol include/e5m2effma.h and include/e5m2effma_ext.h declare
EXPORTS = ("e5ma_gemm", "e5ma_cast", "e5ma_adam", "e5ma_status_string", "e5ma_last_error", "e5ma_quantize",
           "e5ma_gemm_ex", "e5ma_gemm_workspace_size", "e5ma_gemm_noalloc")


class Tensor(ctypes.Structure):
    """e5ma_tensor (include/e5m2effma.h; 48 bytes on LP64)."""
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int), ("scale_inv", ctypes.c_void_p),
                ("scale", ctypes.c_void_p), ("amax", ctypes.c_void_p), ("scaling", ctypes.c_int)]


class AdamConfig(ctypes.Structure):
    """e5ma_adam_config (include/e5m2effma.h; 36 bytes)."""
    _fields_ = [("lr", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float), ("step", ctypes.c_int),
                ("adamw", ctypes.c_int), ("bias_correction", ctypes.c_int), ("grad_scale", ctypes.c_float)]


_lib = None


def lib():
    """The loaded C library (raises when libe5m2effma.so has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                              "g.build()'` (or `make -C e5m2effma_amd/csrc`)")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        TP = ctypes.POINTER(Tensor)
        L.e5ma_gemm.restype = I
        L.e5ma_gemm.argtypes = [I, I, I, I, I, F, TP, I, TP, I, F, TP, I, TP, I, TP, P]
        L.e5ma_gemm_ex.restype = I
        L.e5ma_gemm_ex.argtypes = [I, I, I, I, I, F, TP, I, TP, I, F, TP, I, TP, I, TP, P, S, P]
        L.e5ma_gemm_noalloc.restype = I
        L.e5ma_gemm_noalloc.argtypes = [I, I, I, I, I, F, TP, I, TP, I, F, TP, I, TP, I, TP, P]
        L.e5ma_gemm_workspace_size.restype = I
        L.e5ma_gemm_workspace_size.argtypes = [I, I, I, I, I, I, I, I, I, ctypes.POINTER(S)]
        L.e5ma_cast.restype = I
        L.e5ma_cast.argtypes = [TP, TP, S, P]
        L.e5ma_quantize.restype = I
        L.e5ma_quantize.argtypes = [TP, TP, S, S, F, P, P, P]
        L.e5ma_adam.restype = I
        L.e5ma_adam.argtypes = [ctypes.POINTER(AdamConfig), S, TP, TP, TP, TP, TP, P]
        L.e5ma_status_string.restype = ctypes.c_char_p
        L.e5ma_status_string.argtypes = [I]
        L.e5ma_last_error.restype = ctypes.c_char_p
        L.e5ma_last_error.argtypes = []
        _lib = L
    return _lib


def last_error():
    return lib().e5ma_last_error().decode()


def status_string(s):
    return lib().e5ma_status_string(s).decode()


def tensor(data=None, dtype=FP32, scale_inv=None, scale=None, amax=None, scaling=SCALING_TENSOR):
    """An e5ma_tensor from raw device addresses (ints or None)."""
    return Tensor(data, dtype, scale_inv, scale, amax, scaling)


def ref(t):
    return None if t is None else ctypes.byref(t)


def workspace_size(transa, transb, m, n, k, adt, lda, bdt, ldb):
    """Bytes of split-K workspace e5ma_gemm_ex uses for this GEMM on the current device (0: none)."""
    out = ctypes.c_size_t(0)
    s = lib().e5ma_gemm_workspace_size(transa, transb, m, n, k, adt, lda, bdt, ldb, ctypes.byref(out))
    if s != OK:
        raise RuntimeError(f"e5ma_gemm_workspace_size: {status_string(s)}: {last_error()}")
    return out.value
