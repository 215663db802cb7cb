"""``Float8Tensor`` and ``quantize_linear_``: FP8 weights that ordinary PyTorch code multiplies in FP8.

Interface of the reference's ``binds/python/e5m2effma/tensor.py:26-167``.  A ``Float8Tensor`` is a wrapper
tensor subclass: it reports a nominal high-precision dtype (bfloat16 by default) and the shape of its data,
and holds ``torch.float8_e5m2`` / ``torch.float8_e4m3fn`` codes ``_data`` with their dequantization factor
``_scale_inv`` (value = code * scale_inv): one float32 for the tensor, or one per row (``_scale_dim`` 0) or
per column (1) of a 2-D tensor.  Under ``__torch_dispatch__``:

* ``aten.mm`` / ``aten.addmm`` -- what ``@``, ``torch.matmul``, ``F.linear`` and ``nn.Linear`` lower to --
  run on ``e5ma_gemm`` when every scale is per tensor or along the product's outer dimension;
* ``t`` / ``transpose`` / ``detach`` / ``alias`` / ``clone`` stay FP8 (a transpose moves a per-row scale to
  per-column);
* ``_to_copy`` (``.to(dtype)``, ``.float()``) and every other operation dequantize their FP8 arguments.

Inference only (no autograd).
"""
from typing import Optional

import torch
from torch.utils._pytree import tree_map

_FP8_MAX = {torch.float8_e5m2: 57344.0, torch.float8_e4m3fn: 448.0}
_NOMINAL = (torch.bfloat16, torch.float16, torch.float32)
_aten = torch.ops.aten


class Float8Tensor(torch.Tensor):
    @staticmethod
    def __new__(cls, data: torch.Tensor, scale_inv: torch.Tensor, scale_dim: Optional[int] = None,
                dtype: torch.dtype = torch.bfloat16):
        if data.dtype not in _FP8_MAX:
            raise TypeError(f"Float8Tensor data must be torch.float8_e5m2 or torch.float8_e4m3fn, got {data.dtype}")
        if scale_inv.dtype != torch.float32 or scale_inv.device != data.device:
            raise TypeError("scale_inv must be a float32 tensor on the device of the data")
        if scale_dim is None:
            if scale_inv.numel() != 1:
                raise ValueError(f"a per-tensor scale_inv has one element, got shape {tuple(scale_inv.shape)}")
        else:
            want = data.shape[scale_dim] if data.dim() == 2 and scale_dim in (0, 1) else None
            if want is None or scale_inv.numel() != want:
                raise ValueError(f"scale_dim={scale_dim} needs 2-D data and {want if want is not None else '?'} "
                                 f"factors, got data {tuple(data.shape)} and scale_inv {tuple(scale_inv.shape)}")
        if dtype not in _NOMINAL:
            raise TypeError(f"nominal dtype must be bfloat16, float16 or float32, got {dtype}")
        t = torch.Tensor._make_wrapper_subclass(cls, data.shape, strides=data.stride(), storage_offset=0, dtype=dtype,
                                                device=data.device, requires_grad=False)
        t._data = data
        t._scale_inv = scale_inv.reshape(-1)
        t._scale_dim = scale_dim
        return t

    @classmethod
    def from_float(cls, x: torch.Tensor, *, fp8: torch.dtype = torch.float8_e5m2, per_row: bool = False,
                   dtype: Optional[torch.dtype] = None, margin: float = 1.0) -> "Float8Tensor":
        """Quantize ``x`` with scale = margin * max_finite(fp8) / amax, per tensor or per row of a 2-D ``x``,
        in one ``e5ma_quantize`` call (the reference composes the same steps from torch operations and
        e5ma_cast, tensor.py:60-74).  The nominal dtype defaults to ``x``'s (bfloat16 for other dtypes)."""
        if x.device.type != "cuda":
            raise ValueError("Float8Tensor.from_float needs a tensor on a ROCm device")
        if fp8 not in _FP8_MAX:
            raise TypeError(f"fp8 must be torch.float8_e5m2 or torch.float8_e4m3fn, got {fp8}")
        if dtype is None:
            dtype = x.dtype if x.dtype in _NOMINAL else torch.bfloat16
        if per_row and x.dim() != 2:
            raise ValueError(f"per_row quantization needs a 2-D tensor, got shape {tuple(x.shape)}")
        from . import quantize
        codes, scale_inv, _ = quantize(x.detach(), fp8, per_row=per_row, margin=margin)
        return cls(codes, scale_inv, 0 if per_row else None, dtype)

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        s = self._scale_inv
        if self._scale_dim == 0:
            s = s[:, None]
        elif self._scale_dim == 1:
            s = s[None, :]
        return (self._data.float() * s).to(dtype or self.dtype)

    def __repr__(self):
        how = {None: "per tensor", 0: "per row", 1: "per column"}[self._scale_dim]
        return f"Float8Tensor(shape={tuple(self.shape)}, dtype={self.dtype}, {self._data.dtype}, scale {how})"

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        op = _OPS.get(func)
        if op is not None:
            r = op(*args, **kwargs)
            if r is not NotImplemented:
                return r
        plain = lambda v: v.dequantize() if isinstance(v, Float8Tensor) else v
        return func(*tree_map(plain, args), **tree_map(plain, kwargs))


def _same(x: Float8Tensor, data=None, scale_inv=None, scale_dim="keep"):
    return Float8Tensor(x._data if data is None else data, x._scale_inv if scale_inv is None else scale_inv,
                        x._scale_dim if scale_dim == "keep" else scale_dim, x.dtype)


def _t(x):
    if x.dim() != 2:
        return NotImplemented
    return _same(x, data=x._data.t(), scale_dim=None if x._scale_dim is None else 1 - x._scale_dim)


def _transpose(x, d0, d1):
    if x.dim() != 2 or (d0 % 2) == (d1 % 2):
        return NotImplemented
    return _t(x)


def _operand(x, outer: int):
    """(data, scale_inv, nominal dtype) of a product operand whose outer dimension is ``outer`` (0: rows of
    a, 1: columns of b); None when its scale runs along K, which only dequantization can apply."""
    if not isinstance(x, Float8Tensor):
        return x, None, x.dtype
    if x._scale_dim is not None and x._scale_dim != outer:
        return None
    return x._data, x._scale_inv, x.dtype


def _mm(a, b, bias=None):
    from . import matmul
    pa, pb = _operand(a, 0), _operand(b, 1)
    if pa is None or pb is None or a.dim() != 2 or b.dim() != 2 or a.shape[1] % 16:
        return NotImplemented
    (da, sa, ta), (db, sb, tb) = pa, pb
    ok = (torch.float8_e5m2, torch.float8_e4m3fn, torch.bfloat16, torch.float32)
    if da.dtype not in ok or db.dtype not in ok:
        return NotImplemented  # e.g. a float16 or float64 plain operand: dequantize instead
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != b.shape[1]):
        return NotImplemented  # only a per-column bias vector is fused
    return matmul(da, db, out_dtype=torch.promote_types(ta, tb), bias=bias, scale_a=sa, scale_b=sb)


def _addmm(bias, a, b, *, beta=1, alpha=1):
    if beta != 1 or alpha != 1:
        return NotImplemented
    return _mm(a, b, bias)


def _to_copy(x, dtype=None, device=None, **_):
    y = x.dequantize(dtype)
    return y if device is None else y.to(device)


_OPS = {
    _aten.mm.default: _mm,
    _aten.addmm.default: _addmm,
    _aten.t.default: _t,
    _aten.transpose.int: _transpose,
    _aten.detach.default: lambda x: _same(x),
    _aten.alias.default: lambda x: _same(x),
    _aten.clone.default: lambda x, memory_format=None: _same(x, data=x._data.clone(), scale_inv=x._scale_inv.clone()),
    _aten._to_copy.default: _to_copy,
}


def quantize_linear_(module: torch.nn.Module, *, fp8: torch.dtype = torch.float8_e4m3fn, per_row: bool = True,
                     dtype: Optional[torch.dtype] = None) -> torch.nn.Module:
    """Replace, in place, the weight of every ``nn.Linear`` of ``module`` whose in_features is a multiple of 16
    by a ``Float8Tensor`` (per output feature scales by default; E4M3 by default, whose extra mantissa bit
    suits weights), so its matmuls run in FP8 on ``e5ma_gemm``.  Other layers keep their weights."""
    for m in module.modules():
        if isinstance(m, torch.nn.Linear) and not isinstance(m.weight, Float8Tensor) and m.in_features % 16 == 0:
            w = Float8Tensor.from_float(m.weight.data, fp8=fp8, per_row=per_row, dtype=dtype or m.weight.dtype)
            m.weight = torch.nn.Parameter(w, requires_grad=False)
    return module
