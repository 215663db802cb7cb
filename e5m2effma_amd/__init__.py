"""e5m2effma_amd: FP8 (E5M2 / E4M3) GEMM, GEMV, cast and fused Adam / AdamW on MI355X (gfx950).

A thin PyTorch-ROCm layer over the C ABI of ``include/e5m2effma.h`` (``libe5m2effma.so``), with the
functional interface of the reference's Python package (reference
``binds/python/e5m2effma/__init__.py:58-131``, checks of ``binds/python/csrc/e5m2effma_torch.cpp:127-274``):

* ``matmul(a, b, ...)``: ``out = alpha * (scale_a * scale_b) * (a @ b) + bias + beta * out``;
* ``linear(x, weight, bias, ...)``: ``x @ weight.t() + bias``;
* ``cast(x, dtype, ...)``: element-wise conversion with scale_inv / scale / amax;
* ``quantize(x, dtype, ...)``: FP8 codes with a scale from x's own amax, per tensor or per row;
* ``adam_step(param, grad, exp_avg, exp_avg_sq, ...)``: one fused in-place Adam / AdamW step;
* ``AdamW``: a ``torch.optim`` optimizer on that step (``optim.py``);
* ``Float8Tensor`` / ``quantize_linear_``: FP8 weights with their scale that ``@``, ``F.linear`` and
  ``nn.Linear`` multiply on this library (``tensor.py``).

On import, ``torch.e5m2effma`` (like ``e5m2``) becomes an alias of ``torch.float8_e5m2``, as with the
reference package.

Tensors live on a ROCm device; FP8 tensors use ``torch.float8_e5m2`` / ``torch.float8_e4m3fn`` (OCP,
the encodings of this library).  Scales follow Transformer Engine: ``scale_a`` / ``scale_b`` /
``scale_inv`` dequantize an FP8 input, ``scale_out`` / ``scale`` quantize an FP8 output, ``amax``
tensors receive max |value| before quantization (max-reduced into their content).  Every call runs on
torch's current stream.  Errors: ``TypeError`` (dtype), ``ValueError`` (device, shape, K, overlap, bad
argument), ``NotImplementedError`` (a device other than gfx950), ``RuntimeError`` (runtime failure).
"""
import ctypes
import os
from typing import Optional

import torch

from . import _lib
from ._lib import BF16, E4M3, E5M2, FP16, FP32

__version__ = "0.2.0"
e5m2 = torch.float8_e5m2
e4m3 = torch.float8_e4m3fn
if not hasattr(torch, "e5m2effma"):
    torch.e5m2effma = e5m2
__all__ = ["matmul", "linear", "cast", "quantize", "adam_step", "AdamW", "Float8Tensor", "quantize_linear_", "gemm_raw", "e5m2",
           "e4m3", "torch_ops_enabled", "get_include", "__version__"]

_CODE = {torch.float8_e4m3fn: E4M3, torch.bfloat16: BF16, torch.float16: FP16, torch.float32: FP32,
         torch.float8_e5m2: E5M2}
_FP8 = (torch.float8_e5m2, torch.float8_e4m3fn)
_OPERANDS = (torch.float8_e5m2, torch.float8_e4m3fn, torch.bfloat16, torch.float32)
_OPERANDS_S = "torch.float8_e5m2, torch.float8_e4m3fn, torch.bfloat16 or torch.float32"


def _code(dt, what):
    if dt not in _CODE:
        raise TypeError(f"{what} must be one of torch.float8_e5m2, torch.float8_e4m3fn, torch.bfloat16, "
                        f"torch.float16 or torch.float32, got {dt}")
    return _CODE[dt]


def _check_status(s, what):
    """reference csrc/e5m2effma_torch.cpp:82-88"""
    if s == _lib.OK:
        return
    msg = f"{what} failed ({_lib.status_string(s)}): {_lib.last_error()}"
    if s == _lib.NOT_SUPPORTED:
        raise NotImplementedError(msg)
    if s == _lib.INVALID_VALUE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _check_device(t, dev, what):
    if t.device != dev:
        raise ValueError(f"{what} must be on {dev}, got a tensor on {t.device}")


def _scalar_ptr(t, dev, what):
    if t is None:
        return None
    _check_device(t, dev, what)
    if t.dtype != torch.float32:
        raise TypeError(f"{what} must be torch.float32, got {t.dtype}")
    if t.numel() != 1:
        raise ValueError(f"{what} must have exactly one element, got shape {tuple(t.shape)}")
    return t.data_ptr()


def _operand_scale(t, dev, what, outer, shapes):
    """(pointer, is_vector, holder) of an operand dequantization factor: one float or one per outer index."""
    if t is None:
        return None, False, None
    _check_device(t, dev, what)
    if t.dtype != torch.float32:
        raise TypeError(f"{what} must be torch.float32, got {t.dtype}")
    if t.numel() == 1:
        return t.data_ptr(), False, t
    if t.numel() != outer or t.dim() > 2:
        raise ValueError(f"{what} must have one element (per tensor) or shape {shapes} (one factor per {outer} "
                         f"outer indices), got shape {tuple(t.shape)}")
    h = t.contiguous().view(-1)
    return h.data_ptr(), True, h


def _overlaps(x, y):
    if x.numel() == 0 or y.numel() == 0 or x.untyped_storage().data_ptr() != y.untyped_storage().data_ptr():
        return False
    xs, xe = x.data_ptr(), x.data_ptr() + x.numel() * x.element_size()
    ys, ye = y.data_ptr(), y.data_ptr() + y.numel() * y.element_size()
    return xs < ye and ys < xe


def _layout(t):
    """(ok, row_major, ld) of a 2-D operand as the column-major API sees it (csrc:96-102)."""
    r, c = t.shape
    if t.stride(1) == 1 and (r <= 1 or t.stride(0) >= c):
        return True, True, c if r <= 1 else t.stride(0)
    if t.stride(0) == 1 and (c <= 1 or t.stride(1) >= r):
        return True, False, r if c <= 1 else t.stride(1)
    return False, False, 0


def _qualified(t, k_is_dim1):
    """The operand as is when the library can read it, else a K-contiguous copy (csrc:106-113)."""
    ok, rm, ld = _layout(t)
    if ok and ld % 16 == 0 and t.data_ptr() % 16 == 0:
        return t, rm, ld
    c = t.contiguous() if k_is_dim1 else t.t().contiguous().t()
    _, rm, ld = _layout(c)
    return c, rm, ld


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check_gpu(dev):
    if dev.type != "cuda":
        raise ValueError(f"expected a tensor on a ROCm device, got one on {dev}")


def matmul(a: torch.Tensor, b: torch.Tensor, *, out_dtype: Optional[torch.dtype] = None,
           bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None, alpha: float = 1.0,
           beta: float = 0.0, scale_a: Optional[torch.Tensor] = None, scale_b: Optional[torch.Tensor] = None,
           scale_out: Optional[torch.Tensor] = None, amax_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row-major ``out [M, N] = alpha * (scale_a * scale_b) * (a [M, K] @ b [K, N]) + bias + beta * out``.

    Issued to the column-major C ABI as ``out^T = b^T a^T`` (reference csrc/e5m2effma_torch.cpp:127-200):
    ``b`` becomes operand A, ``a`` operand B; a row-wise ``scale_a`` [M] is the per-column scale of
    op(B), ``scale_b`` [N] the per-row scale of op(A).  With M <= 8, ``a`` row-contiguous and ``b`` a
    column-contiguous FP8 matrix (``W.t()``), the GEMV kernel runs.
    """
    if not isinstance(a, torch.Tensor) or not isinstance(b, torch.Tensor):
        raise TypeError("a and b must be tensors")
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError(f"a and b must be 2-D, got shapes {tuple(a.shape)} and {tuple(b.shape)}")
    for t, nm in ((a, "a"), (b, "b")):
        if t.dtype not in _OPERANDS:
            raise TypeError(f"{nm} must be {_OPERANDS_S}, got {t.dtype}")
    _check_gpu(a.device)
    dev = a.device
    _check_device(b, dev, "b")
    M, K, N = a.shape[0], a.shape[1], b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"shapes do not match for a @ b: {tuple(a.shape)} and {tuple(b.shape)}")
    if K % 16:
        raise ValueError(f"K = {K} must be a multiple of 16 (pad the reduction dimension with zeros)")
    if scale_a is not None and a.dtype not in _FP8:
        raise ValueError("scale_a is only meaningful for an FP8 a (it is the dequantization factor)")
    if scale_b is not None and b.dtype not in _FP8:
        raise ValueError("scale_b is only meaningful for an FP8 b (it is the dequantization factor)")
    if beta != 0.0 and out is None:
        raise ValueError("beta != 0 accumulates into out, so out must be given")
    if out is not None:
        _check_device(out, dev, "out")
        _code(out.dtype, "out")
        if out_dtype is not None and out_dtype != out.dtype:
            raise ValueError(f"out_dtype {out_dtype} does not match out.dtype {out.dtype}")
        if out.dim() != 2 or tuple(out.shape) != (M, N):
            raise ValueError(f"out must have shape [{M}, {N}], got {tuple(out.shape)}")
        if out.stride(1) != 1 or (M > 1 and out.stride(0) < N):
            raise ValueError(f"out must be row-contiguous (stride(1) == 1), got strides {out.stride()}")
        for t, nm in ((a, "a"), (b, "b")):
            if _overlaps(out, t):
                raise ValueError(f"out must not share memory with {nm}")
    else:
        out = torch.empty((M, N), dtype=out_dtype or torch.bfloat16, device=dev)
    dt = _code(out.dtype, "out")
    if scale_out is not None and out.dtype not in _FP8:
        raise ValueError("scale_out is only meaningful for an FP8 output (it is the quantization factor)")
    if bias is not None:
        _check_device(bias, dev, "bias")
        _code(bias.dtype, "bias")
        if bias.dim() != 1 or bias.shape[0] != N or bias.stride(0) != 1:
            raise ValueError(f"bias must be a contiguous vector of length N = {N}, got shape {tuple(bias.shape)}")
    if M == 0 or N == 0:
        return out
    qa, a_rm, lda_ = _qualified(a, True)
    qb, b_rm, ldb_ = _qualified(b, False)
    transa = _lib.OP_N if b_rm else _lib.OP_T
    transb = _lib.OP_N if a_rm else _lib.OP_T
    with torch.cuda.device(dev):
        sa_p, sa_vec, _ha = _operand_scale(scale_a, dev, "scale_a", M, "[M] or [M, 1]")
        sb_p, sb_vec, _hb = _operand_scale(scale_b, dev, "scale_b", N, "[N] or [1, N]")
        A = _lib.tensor(qb.data_ptr(), _CODE[b.dtype], sb_p, None, None, int(sb_vec))
        B = _lib.tensor(qa.data_ptr(), _CODE[a.dtype], sa_p, None, None, int(sa_vec))
        D = _lib.tensor(out.data_ptr(), dt, None, _scalar_ptr(scale_out, dev, "scale_out"),
                        _scalar_ptr(amax_out, dev, "amax_out"))
        BIAS = _lib.tensor(bias.data_ptr(), _CODE[bias.dtype]) if bias is not None else None
        ldd = N if M <= 1 else out.stride(0)
        # split-K workspace for small grids from torch's allocator, freed in stream order after the call
        ws_bytes = _lib.workspace_size(transa, transb, N, M, K, _CODE[b.dtype], ldb_, _CODE[a.dtype], lda_)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        s = _lib.lib().e5ma_gemm_ex(transa, transb, N, M, K, float(alpha), ctypes.byref(A), ldb_, ctypes.byref(B),
                                    lda_, float(beta), None, 0, ctypes.byref(D), ldd, _lib.ref(BIAS),
                                    None if ws is None else ws.data_ptr(), ws_bytes, _stream())
    _check_status(s, "e5ma_gemm_ex")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
           out_dtype: Optional[torch.dtype] = None, scale_x: Optional[torch.Tensor] = None,
           scale_w: Optional[torch.Tensor] = None, scale_out: Optional[torch.Tensor] = None,
           amax_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x @ weight.t() + bias`` (reference ``__init__.py:80-101``): ``x`` [..., K], ``weight`` [N, K]."""
    if not isinstance(x, torch.Tensor) or not isinstance(weight, torch.Tensor):
        raise TypeError("x and weight must be tensors")
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [out_features, in_features], got shape {tuple(weight.shape)}")
    if x.dim() < 1 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"x must have shape [..., {weight.shape[1]}], got {tuple(x.shape)}")
    x2 = x.reshape(-1, x.shape[-1])
    if scale_x is not None and scale_x.numel() > 1:
        scale_x = scale_x.reshape(-1)
    y = matmul(x2, weight.t(), out_dtype=out_dtype, bias=bias, scale_a=scale_x, scale_b=scale_w,
               scale_out=scale_out, amax_out=amax_out)
    return y.reshape(*x.shape[:-1], weight.shape[0])


def cast(x: torch.Tensor, dtype: torch.dtype, *, scale_inv: Optional[torch.Tensor] = None,
         scale: Optional[torch.Tensor] = None, amax: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Element-wise conversion between the five dtypes (reference ``__init__.py:104-114``,
    csrc/e5m2effma_torch.cpp:203-219): ``value = x * scale_inv`` (FP8 x), result RNE-satfinite of
    ``value * scale`` (FP8 dtype) or RNE, ``amax`` gets max |value|."""
    _check_gpu(x.device)
    dev = x.device
    st, dt = _code(x.dtype, "x"), _code(dtype, "dtype")
    if scale_inv is not None and x.dtype not in _FP8:
        raise ValueError("scale_inv is only meaningful for an FP8 x")
    if scale is not None and dtype not in _FP8:
        raise ValueError("scale is only meaningful for an FP8 result")
    xc = x.contiguous()
    y = torch.empty(xc.shape, dtype=dtype, device=dev)
    if xc.numel() == 0:
        return y
    with torch.cuda.device(dev):
        S = _lib.tensor(xc.data_ptr(), st, _scalar_ptr(scale_inv, dev, "scale_inv"))
        D = _lib.tensor(y.data_ptr(), dt, None, _scalar_ptr(scale, dev, "scale"), _scalar_ptr(amax, dev, "amax"))
        s = _lib.lib().e5ma_cast(ctypes.byref(S), ctypes.byref(D), xc.numel(), _stream())
    _check_status(s, "e5ma_cast")
    return y


def quantize(x: torch.Tensor, dtype: torch.dtype = torch.float8_e5m2, *, per_row: bool = False, margin: float = 1.0,
             scale_inv: Optional[torch.Tensor] = None):
    """FP8 codes of ``x`` with a scale from its own amax, per tensor or per row of a 2-D ``x``, on
    ``e5ma_quantize`` (include/e5m2effma_ext.h): the steps of the reference's
    ``Float8Tensor.from_float`` (``tensor.py:60-74``) in one call.  ``scale = margin * max_finite / amax``
    (amax clamped to 1e-12), codes RNE-satfinite of ``x * scale``.  Returns ``(codes, scale_inv, amax)``,
    the last two float32 of shape (1,) or (rows,).  ``scale_inv`` dequantizes an FP8 ``x``."""
    _check_gpu(x.device)
    dev = x.device
    st = _code(x.dtype, "x")
    if dtype not in _FP8:
        raise TypeError(f"dtype must be torch.float8_e5m2 or torch.float8_e4m3fn, got {dtype}")
    if scale_inv is not None and x.dtype not in _FP8:
        raise ValueError("scale_inv is only meaningful for an FP8 x")
    if per_row and x.dim() != 2:
        raise ValueError(f"per_row quantization needs a 2-D tensor, got shape {tuple(x.shape)}")
    if not margin > 0:
        raise ValueError(f"margin must be positive, got {margin}")
    xc = x.contiguous()
    rows, cols = (xc.shape[0], xc.shape[1]) if per_row else (1, xc.numel())
    groups = rows if per_row else 1
    codes = torch.empty(xc.shape, dtype=dtype, device=dev)
    sinv = torch.empty(groups, dtype=torch.float32, device=dev)
    amax = torch.empty(groups, dtype=torch.float32, device=dev)
    qmax = float(torch.tensor(margin * (57344.0 if dtype == torch.float8_e5m2 else 448.0), dtype=torch.float32))
    if xc.numel() == 0:
        return codes, sinv.fill_(float("nan")), amax.zero_()
    with torch.cuda.device(dev):
        S = _lib.tensor(xc.data_ptr(), st, _scalar_ptr(scale_inv, dev, "scale_inv"))
        D = _lib.tensor(codes.data_ptr(), _CODE[dtype], scaling=_lib.SCALING_OUTER if per_row else _lib.SCALING_TENSOR)
        s = _lib.lib().e5ma_quantize(ctypes.byref(S), ctypes.byref(D), rows, cols, qmax, sinv.data_ptr(),
                                     amax.data_ptr(), _stream())
    _check_status(s, "e5ma_quantize")
    return codes, sinv, amax


def adam_step(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor, *,
              lr: float, betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 0.0, step: int,
              adamw: bool = True, bias_correction: bool = True, grad_scale: float = 1.0,
              param_fp8: Optional[torch.Tensor] = None, fp8_scale: Optional[torch.Tensor] = None,
              fp8_amax: Optional[torch.Tensor] = None) -> None:
    """One fused in-place Adam / AdamW step, ``step`` 1-based (reference ``__init__.py:117-131``,
    csrc/e5m2effma_torch.cpp:222-274)."""
    beta1, beta2 = betas
    _check_gpu(param.device)
    dev = param.device
    for t, nm in ((grad, "grad"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        _check_device(t, dev, nm)
    if param.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"param must be torch.float32 or torch.bfloat16, got {param.dtype}")
    if grad.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"grad must be torch.float32, torch.bfloat16 or torch.float16, got {grad.dtype}")
    if exp_avg.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"exp_avg must be torch.float32 or torch.bfloat16, got {exp_avg.dtype}")
    if exp_avg_sq.dtype != exp_avg.dtype:
        raise TypeError(f"exp_avg_sq must have the dtype of exp_avg ({exp_avg.dtype}), got {exp_avg_sq.dtype}")
    n = param.numel()
    for t, nm in ((grad, "grad"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if t.numel() != n:
            raise ValueError(f"{nm} has {t.numel()} elements, param has {n}")
    for t, nm in ((param, "param"), (grad, "grad"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    if grad.is_sparse:
        raise ValueError("sparse gradients are not supported")
    if not (1 <= step <= 2**31 - 1):
        raise ValueError(f"step must be >= 1 (1-based), got {step}")
    if lr < 0 or eps < 0 or weight_decay < 0:
        raise ValueError("lr, eps and weight_decay must be non-negative")
    if not (0 <= beta1 < 1 and 0 <= beta2 < 1):
        raise ValueError(f"betas must be in [0, 1), got ({beta1}, {beta2})")
    for x, y, nx, ny in ((exp_avg, exp_avg_sq, "exp_avg", "exp_avg_sq"), (param, exp_avg, "param", "exp_avg"),
                         (param, exp_avg_sq, "param", "exp_avg_sq")):
        if _overlaps(x, y):
            raise ValueError(f"{nx} must not share memory with {ny}")
    if param_fp8 is not None:
        _check_device(param_fp8, dev, "param_fp8")
        if param_fp8.dtype not in _FP8:
            raise TypeError(f"param_fp8 must be torch.float8_e5m2 or torch.float8_e4m3fn, got {param_fp8.dtype}")
        if param_fp8.numel() != n or not param_fp8.is_contiguous():
            raise ValueError(f"param_fp8 must be contiguous with the element count of param ({n})")
    elif fp8_scale is not None or fp8_amax is not None:
        raise ValueError("fp8_scale / fp8_amax need param_fp8")
    if n == 0:
        return
    with torch.cuda.device(dev):
        cfg = _lib.AdamConfig(lr, beta1, beta2, eps, weight_decay, int(step), int(bool(adamw)),
                              int(bool(bias_correction)), grad_scale)
        P = _lib.tensor(param.data_ptr(), _CODE[param.dtype])
        G = _lib.tensor(grad.data_ptr(), _CODE[grad.dtype])
        Mo = _lib.tensor(exp_avg.data_ptr(), _CODE[exp_avg.dtype])
        V = _lib.tensor(exp_avg_sq.data_ptr(), _CODE[exp_avg_sq.dtype])
        Q = None
        if param_fp8 is not None:
            Q = _lib.tensor(param_fp8.data_ptr(), _CODE[param_fp8.dtype], None,
                            _scalar_ptr(fp8_scale, dev, "fp8_scale"), _scalar_ptr(fp8_amax, dev, "fp8_amax"))
        s = _lib.lib().e5ma_adam(ctypes.byref(cfg), n, ctypes.byref(P), ctypes.byref(G), ctypes.byref(Mo),
                                 ctypes.byref(V), _lib.ref(Q), _stream())
    _check_status(s, "e5ma_adam")


def get_include() -> list:
    """Directories for HIP code that builds on this library (reference ``__init__.py:49-55``): the C ABI
    headers (``e5m2effma.h``, ``e5m2effma_ext.h``) and the device-side codecs ``e5ma_device.hpp`` (FP8 decode,
    RNE / saturating encode, typed loads and stores; gfx950 only).  Compile with ``-I`` on both; code built
    from them is consistent with this version of the library only."""
    here = os.path.dirname(os.path.abspath(__file__))
    return [os.path.join(os.path.dirname(here), "include"), os.path.join(here, "csrc")]


def torch_ops_enabled() -> bool:
    """Whether ``torch._scaled_mm`` runs on this library in this process: never.  The reference overrides
    ``aten::_scaled_mm`` only on GPUs without native FP8 and keeps PyTorch's kernel elsewhere (reference
    ``__init__.py:165-170``); gfx950 has native FP8 in PyTorch's own ``_scaled_mm``, so nothing is
    overridden here."""
    return False


def gemm_raw(transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, D, ldd, bias=None, stream=None):
    """e5ma_gemm on e5ma_tensor descriptors (``_lib.Tensor``), column-major as the C ABI; returns the status."""
    st = _stream() if stream is None else ctypes.c_void_p(stream)
    return _lib.lib().e5ma_gemm(transa, transb, m, n, k, float(alpha), _lib.ref(A), lda, _lib.ref(B), ldb,
                                float(beta), _lib.ref(C), ldc, _lib.ref(D), ldd, _lib.ref(bias), st)


from .optim import AdamW  # noqa: E402  (they call the functions above)
from .tensor import Float8Tensor, quantize_linear_  # noqa: E402
