"""CPU oracle of the reference's FP8 compute semantics -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
package, as the checker or as the timed CPU baseline.  The product (``e5m2effma_amd``) never does.

The arithmetic lives in ``e5ma_oracle.c`` (built into ``liboracle.so`` by ``oracle/Makefile``); each C
function cites the reference file:line it restates.  This module only marshals numpy arrays.
``ref_library()`` loads ``_ref/libref.so``: the reference's own exact MAC model
(``tests/e5m2effma_ref.h`` via ``tests/ref_capi.cpp``), compiled from the reference sources where
they lie, when they were present at build time.
"""
import ctypes
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
E4M3, BF16, FP16, FP32, E5M2 = 0, 1, 2, 3, 4
NP_DTYPE = {E4M3: np.uint8, E5M2: np.uint8, BF16: np.uint16, FP16: np.uint16, FP32: np.float32}
ESIZE = {E4M3: 1, E5M2: 1, BF16: 2, FP16: 2, FP32: 4}

_lib = None
_lock = threading.Lock()


def build():
    """Compile liboracle.so (and _ref/libref.so when the reference sources exist)."""
    import subprocess
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("transa", ctypes.c_int), ("transb", ctypes.c_int), ("m", ctypes.c_int), ("n", ctypes.c_int),
        ("k", ctypes.c_int), ("alpha", ctypes.c_float),
        ("adt", ctypes.c_int), ("A", ctypes.c_void_p), ("lda", ctypes.c_int), ("sa", ctypes.c_void_p),
        ("sa_vec", ctypes.c_int),
        ("bdt", ctypes.c_int), ("B", ctypes.c_void_p), ("ldb", ctypes.c_int), ("sb", ctypes.c_void_p),
        ("sb_vec", ctypes.c_int),
        ("beta", ctypes.c_float),
        ("cdt", ctypes.c_int), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int), ("csinv", ctypes.c_float),
        ("ddt", ctypes.c_int), ("D", ctypes.c_void_p), ("ldd", ctypes.c_int), ("qscale", ctypes.c_float),
        ("biasdt", ctypes.c_int), ("bias", ctypes.c_void_p),
        ("ocp_operands", ctypes.c_int),
    ]


class AdamConfig(ctypes.Structure):
    _fields_ = [("lr", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float), ("step", ctypes.c_int),
                ("adamw", ctypes.c_int), ("bias_correction", ctypes.c_int), ("grad_scale", ctypes.c_float)]


def lib():
    global _lib
    with _lock:
        if _lib is None:
            path = os.path.join(HERE, "liboracle.so")
            if not os.path.exists(path):
                build()
            L = ctypes.CDLL(path)
            vp, sz, f, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int
            u8, u16, u32 = ctypes.c_uint8, ctypes.c_uint16, ctypes.c_uint32
            sig = {
                "orc_e4m3_value": (f, [u8]), "orc_e5m2_value": (f, [u8]),
                "orc_e4m3_operand": (f, [u8]), "orc_e5m2_operand": (f, [u8]),
                "orc_bf16_value": (f, [u16]), "orc_f16_value": (f, [u16]),
                "orc_f32_to_bf16": (u16, [f]), "orc_f32_to_f16": (u16, [f]),
                "orc_f32_to_e4m3": (u8, [f]), "orc_f32_to_e5m2": (u8, [f]),
                "orc_fp8_encode_search": (u8, [f, i]),
                "orc_lane": (u16, [u8, u8, u16, i, i]),
                "orc_encode_batch": (None, [i, vp, vp, sz, f]),
                "orc_decode_batch": (None, [i, vp, vp, sz, f]),
                "orc_lane_batch": (None, [vp, vp, vp, i, i, vp, sz]),
                "orc_lane_compare": (sz, [vp, vp, sz, i, i, vp]),
                "orc_lane_sweep": (None, [vp, vp, sz, i, i, vp]),
                "orc_lane_gemm": (None, [vp, vp, vp, i, i, i, i, vp, i, i]),
                "orc_encode_selfcheck": (sz, [i, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, vp]),
                "orc_cast": (f, [i, i, vp, vp, sz, f, f, f]),
                "orc_quantize": (None, [i, i, vp, vp, sz, sz, f, f, i, vp, vp]),
                "orc_gemm_chain": (f, [vp, f, i, i, i]),
                "orc_gemm_exact": (None, [vp, vp, vp, sz, vp, vp]),
                "orc_gemm_check": (sz, [vp, vp, vp, vp, vp, sz, ctypes.c_double, vp, vp, vp]),
                "orc_adam": (f, [vp, sz, i, vp, i, vp, i, vp, vp, i, vp, f, f, sz, sz]),
            }
            for name, (res, args) in sig.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def ref_library():
    """ctypes handle of the reference's exact MAC model, or None when it was not built."""
    path = os.path.join(HERE, "_ref", "libref.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    L.ref_lane.restype = ctypes.c_uint32
    L.ref_lane.argtypes = [ctypes.c_uint32] * 3 + [ctypes.c_int] * 2
    return L


# ---- element codecs ------------------------------------------------------------------------------
def encode(dtype, x, qscale=1.0):
    """float32 array -> codes of ``dtype`` (store_any semantics, FP8: RNE satfinite of x * qscale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=NP_DTYPE[dtype])
    lib().orc_encode_batch(dtype, _p(x), _p(out), x.size, qscale)
    return out


def decode(dtype, codes, sinv=1.0):
    """codes of ``dtype`` -> float32 values (load_any semantics, FP8 times sinv)."""
    codes = np.ascontiguousarray(codes, dtype=NP_DTYPE[dtype])
    out = np.empty(codes.shape, dtype=np.float32)
    lib().orc_decode_batch(dtype, _p(codes), _p(out), codes.size, sinv)
    return out


def lane(a, b, acc, fa, fb):
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8)
    acc = np.ascontiguousarray(acc, np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().orc_lane_batch(_p(a), _p(b), _p(acc), fa, fb, _p(out), a.size)
    return out


def lane_sweep(accs, fa, fb, fn=None):
    """Outputs of a lane function (default: the oracle's) over all 65536 FP8 pairs per accumulator:
    array [len(accs), 256, 256] of BF16 bits.  fn: a ctypes function pointer (e.g. ref_lane)."""
    accs = np.ascontiguousarray(accs, np.uint16)
    out = np.empty((accs.size, 256, 256), np.uint16)
    ptr = None if fn is None else ctypes.cast(fn, ctypes.c_void_p)
    lib().orc_lane_sweep(ptr, _p(accs), accs.size, fa, fb, _p(out))
    return out


def lane_gemm(a, b, M, N, K, fa, fb, fn=None, rows=None, threads=1):
    """BASELINE config 1's CPU path: row-major a (M x K) times b (K x N), FP8 codes of formats fa / fb
    (1 = E5M2), as a BF16-accumulating chain of a lane function over k (default: the oracle's; fn: a
    ctypes function pointer such as the reference's ref_lane).  Returns the BF16 bits of rows
    rows[0] .. rows[1] - 1 (all rows by default), computed by `threads` threads."""
    r0, r1 = (0, M) if rows is None else rows
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8)
    out = np.zeros(M * N, np.uint16)
    ptr = None if fn is None else ctypes.cast(fn, ctypes.c_void_p)
    bounds = np.linspace(r0, r1, max(1, min(threads, r1 - r0)) + 1).astype(np.int64)

    def work(t):
        lib().orc_lane_gemm(ptr, _p(a), _p(b), N, K, fa, fb, _p(out), int(bounds[t]), int(bounds[t + 1]))
    ths = [threading.Thread(target=work, args=(t,)) for t in range(len(bounds) - 1)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    return out.reshape(M, N)[r0:r1]


def cast(tin, tout, src, count, sinv=1.0, qscale=1.0, amax_in=0.0):
    dst = np.empty(count, dtype=NP_DTYPE[tout])
    amax = lib().orc_cast(tin, tout, _p(np.ascontiguousarray(src)), _p(dst), count, sinv, qscale, amax_in)
    return dst, amax


def quantize(tin, tout, src, rows, cols, qmax, per_row=False, sinv=1.0):
    """Float8Tensor.from_float's quantization of a rows x cols row-major ``src`` (codes of ``tin``):
    returns (codes, scale_inv, amax), one scale per tensor or per row."""
    groups = rows if per_row else 1
    dst = np.empty(rows * cols, dtype=NP_DTYPE[tout])
    sc = np.empty(groups, np.float32)
    am = np.empty(groups, np.float32)
    lib().orc_quantize(tin, tout, _p(np.ascontiguousarray(src)), _p(dst), rows, cols, sinv, qmax, int(per_row),
                       _p(sc), _p(am))
    return dst, sc, am


# ---- GEMM ----------------------------------------------------------------------------------------
class Gemm:
    """One e5ma_gemm call over numpy buffers (column-major, the C API's argument meaning)."""

    def __init__(self, transa, transb, m, n, k, alpha, adt, A, lda, bdt, B, ldb, *, sa=None, sa_vec=False,
                 sb=None, sb_vec=False, beta=0.0, cdt=None, C=None, ldc=0, csinv=1.0, ddt=BF16, D=None,
                 ldd=None, qscale=1.0, biasdt=FP32, bias=None, ocp_operands=False):
        self.keep = []
        ldd = m if ldd is None else ldd
        if D is None:
            D = np.zeros(ldd * n, dtype=NP_DTYPE[ddt])
        self.D = D

        def arr(x, dt=None):
            if x is None:
                return None
            x = np.ascontiguousarray(x if dt is None else np.asarray(x, dtype=dt))
            self.keep.append(x)
            return x
        self.sa, self.sb = arr(sa, np.float32), arr(sb, np.float32)
        self.A, self.B, self.C, self.bias = arr(A), arr(B), arr(C), arr(bias)
        self.args = GemmArgs(transa, transb, m, n, k, alpha, adt, _p(self.A), lda, _p(self.sa), int(sa_vec),
                             bdt, _p(self.B), ldb, _p(self.sb), int(sb_vec), beta,
                             ddt if cdt is None else cdt, _p(self.C), ldc, csinv,
                             ddt, _p(self.D), ldd, qscale, biasdt, _p(self.bias), int(ocp_operands))

    def chain(self, amax_in=0.0, rows=None, threads=1):
        """The reference tiled kernel's ascending-k FFMA chain, writing self.D; returns amax."""
        r0, r1 = (0, self.args.m) if rows is None else rows
        return lib().orc_gemm_chain(ctypes.byref(self.args), amax_in, r0, r1, threads)

    def exact(self, iis, jjs):
        iis = np.ascontiguousarray(iis, np.int32)
        jjs = np.ascontiguousarray(jjs, np.int32)
        ex = np.empty(iis.size, np.float64)
        mag = np.empty(iis.size, np.float64)
        lib().orc_gemm_exact(ctypes.byref(self.args), _p(iis), _p(jjs), iis.size, _p(ex), _p(mag))
        return ex, mag

    def check(self, D_got, C_before, iis, jjs, err_factor=2.0, threads=8):
        """Count outputs outside the bound; returns (bad, first_bad_index, amax_lo, amax_hi)."""
        iis = np.ascontiguousarray(iis, np.int32)
        jjs = np.ascontiguousarray(jjs, np.int32)
        D_got = np.ascontiguousarray(D_got)
        Cb = None if C_before is None else np.ascontiguousarray(C_before)
        n = iis.size
        parts = max(1, min(threads, n // 256))
        bounds = np.linspace(0, n, parts + 1).astype(np.int64)
        res = [None] * parts

        def work(t):
            lo, hi = int(bounds[t]), int(bounds[t + 1])
            alo, ahi, fb = ctypes.c_float(0), ctypes.c_float(0), ctypes.c_int64(-1)
            bad = lib().orc_gemm_check(ctypes.byref(self.args), _p(D_got), _p(Cb), _p(iis[lo:hi]), _p(jjs[lo:hi]),
                                       hi - lo, err_factor, ctypes.byref(alo), ctypes.byref(ahi), ctypes.byref(fb))
            res[t] = (bad, lo + fb.value if fb.value >= 0 else -1, alo.value, ahi.value)
        ths = [threading.Thread(target=work, args=(t,)) for t in range(parts)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        bad = sum(r[0] for r in res)
        firsts = [r[1] for r in res if r[1] >= 0]
        return bad, (firsts[0] if firsts else -1), max(r[2] for r in res), max(r[3] for r in res)


# ---- Adam ----------------------------------------------------------------------------------------
def adam(cfg, pdt, p, gdt, g, mdt, m, v, qdt=E5M2, q=None, qscale=1.0, amax_in=0.0, threads=1):
    """In-place Adam / AdamW step over numpy buffers (elementwise; threads split the range)."""
    if isinstance(cfg, dict):
        cfg = AdamConfig(**cfg)
    count = p.size
    parts = max(1, min(threads, count // 65536))
    bounds = np.linspace(0, count, parts + 1).astype(np.int64)
    res = [amax_in] * parts

    def work(t):
        res[t] = lib().orc_adam(ctypes.byref(cfg), count, pdt, _p(p), gdt, _p(g), mdt, _p(m), _p(v), qdt, _p(q),
                                qscale, amax_in, int(bounds[t]), int(bounds[t + 1]))
    ths = [threading.Thread(target=work, args=(t,)) for t in range(parts)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    out = amax_in
    for r in res:  # every part started from amax_in; merge with the integer rule
        if np.float32(r).view(np.int32) > np.float32(out).view(np.int32):
            out = r
    return float(out)


def f32_bits(x):
    return np.asarray(x, np.float32).view(np.uint32)
