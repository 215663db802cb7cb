"""``Float8Tensor``: FP8 codes plus their dequantization scale behind an ordinary tensor interface.

The reference package's tensor subclass (reference ``binds/python/e5m2effma/tensor.py:26-167``) lets
unmodified PyTorch code run its matrix products in FP8: the tensor reports a high-precision dtype and
shape while it stores ``torch.float8_e5m2`` / ``torch.float8_e4m3fn`` codes and ``scale_inv``
(value = code * scale_inv), one factor for the tensor or one per row / column of a 2-D tensor.

Here the stored form is a ``Codes`` record and every aten call the subclass sees falls in one of four
kinds (``_kind``):

* ``product`` -- ``mm`` / ``addmm`` (``@``, ``torch.matmul``, ``F.linear`` and ``nn.Linear`` end there):
  one ``e5ma_gemm_ex`` call through :func:`e5m2effma_amd.matmul`, the scales applied in the epilogue;
* ``relayout`` -- ``t``, ``transpose``, ``permute`` of a 2-D tensor: the same codes, transposed view,
  the scale axis swapped;
* ``alias`` / ``copy`` -- ``detach``, ``alias`` share the codes, ``clone`` copies them;
* everything else dequantizes its Float8Tensor arguments and runs in the nominal dtype (``_to_copy``,
  i.e. ``.to()`` / ``.float()``, included).

A product falls back to dequantization when the library cannot apply an operand's scale in the epilogue
(a scale that varies along K), when K is not a multiple of 16, or for operands the GEMM does not take.
Inference only: no autograd (``requires_grad=False``).
"""
from typing import NamedTuple, Optional

import torch
import torch.utils._pytree as pytree

__all__ = ["Float8Tensor", "quantize_linear_"]

_QMAX = {torch.float8_e5m2: 57344.0, torch.float8_e4m3fn: 448.0}  # largest finite value per format
_NOMINAL = (torch.bfloat16, torch.float16, torch.float32)
_aten = torch.ops.aten


class Codes(NamedTuple):
    """FP8 codes and their dequantization factors: ``axis`` None (one factor), 0 (one per row) or 1
    (one per column of a 2-D tensor)."""
    data: torch.Tensor
    scale_inv: torch.Tensor
    axis: Optional[int]

    def value(self, dtype):
        s = self.scale_inv
        if self.axis == 0:
            s = s.reshape(-1, 1)
        elif self.axis == 1:
            s = s.reshape(1, -1)
        return (self.data.to(torch.float32) * s).to(dtype)

    def transposed(self):
        return Codes(self.data.t(), self.scale_inv, None if self.axis is None else 1 - self.axis)


def _check_codes(data, scale_inv, axis, dtype):
    if data.dtype not in _QMAX:
        raise TypeError(f"Float8Tensor holds torch.float8_e5m2 or torch.float8_e4m3fn codes, not {data.dtype}")
    if scale_inv.dtype != torch.float32:
        raise TypeError(f"scale_inv must be a torch.float32 tensor, got {scale_inv.dtype}")
    if scale_inv.device != data.device:
        raise TypeError(f"scale_inv is on {scale_inv.device}, the codes on {data.device}")
    if dtype not in _NOMINAL:
        raise TypeError(f"the nominal dtype must be torch.bfloat16, torch.float16 or torch.float32, not {dtype}")
    if axis is None:
        if scale_inv.numel() != 1:
            raise ValueError(f"a per-tensor scale_inv has one element, got {scale_inv.numel()}")
        return
    if axis not in (0, 1) or data.dim() != 2:
        raise ValueError(f"scale_dim {axis} needs 2-D codes and must be 0 (rows) or 1 (columns); codes have shape "
                         f"{tuple(data.shape)}")
    if scale_inv.numel() != data.shape[axis]:
        raise ValueError(f"scale_dim {axis} needs {data.shape[axis]} factors, got {scale_inv.numel()}")


class Float8Tensor(torch.Tensor):
    """FP8 codes with their dequantization factors, presented as a tensor of the nominal ``dtype``.

    ``Float8Tensor(data, scale_inv, scale_dim=None, dtype=torch.bfloat16)``: ``data`` float8 codes,
    ``scale_inv`` float32 (one element, or with ``scale_dim`` 0 / 1 one per row / column of 2-D data).
    """

    @staticmethod
    def __new__(cls, data: torch.Tensor, scale_inv: torch.Tensor, scale_dim: Optional[int] = None,
                dtype: torch.dtype = torch.bfloat16):
        _check_codes(data, scale_inv, scale_dim, dtype)
        t = torch.Tensor._make_wrapper_subclass(cls, data.shape, strides=data.stride(), storage_offset=0,
                                                dtype=dtype, device=data.device, requires_grad=False)
        t._codes = Codes(data, scale_inv.reshape(-1), scale_dim)
        return t

    @classmethod
    def _wrap(cls, codes: Codes, dtype):
        return cls(codes.data, codes.scale_inv, codes.axis, dtype)

    # ---- the stored form ------------------------------------------------------------------------
    @property
    def codes(self) -> torch.Tensor:
        """The float8 codes."""
        return self._codes.data

    @property
    def scale_inv(self) -> torch.Tensor:
        """Dequantization factors (float32): one, or one per row / column (``scale_dim``)."""
        return self._codes.scale_inv

    @property
    def scale_dim(self) -> Optional[int]:
        return self._codes.axis

    # the reference package's attribute names
    _data = codes
    _scale_inv = scale_inv
    _scale_dim = scale_dim

    @classmethod
    def from_float(cls, x: torch.Tensor, *, fp8: torch.dtype = torch.float8_e5m2, per_row: bool = False,
                   dtype: Optional[torch.dtype] = None, margin: float = 1.0) -> "Float8Tensor":
        """Quantize ``x`` with the scale of its own amax: ``scale = margin * max_finite(fp8) / amax``, per
        tensor or per row of a 2-D ``x``, in one ``e5ma_quantize`` call (bit-identical to the reference's
        torch steps, reference ``tensor.py:60-74``).  The nominal dtype defaults to ``x``'s when that is
        BF16 / FP16 / FP32, else BF16."""
        from . import quantize
        if fp8 not in _QMAX:
            raise TypeError(f"fp8 must be torch.float8_e5m2 or torch.float8_e4m3fn, got {fp8}")
        if x.device.type != "cuda":
            raise ValueError(f"Float8Tensor.from_float quantizes on a ROCm device; x is on {x.device}")
        codes, sinv, _ = quantize(x.detach(), fp8, per_row=per_row, margin=margin)
        nominal = dtype or (x.dtype if x.dtype in _NOMINAL else torch.bfloat16)
        return cls(codes, sinv, 0 if per_row else None, nominal)

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """The values ``code * scale_inv`` as an ordinary tensor (nominal dtype by default)."""
        return self._codes.value(dtype or self.dtype)

    def __repr__(self):
        where = {None: "per tensor", 0: "per row", 1: "per column"}[self._codes.axis]
        return (f"Float8Tensor({self._codes.data.dtype}, shape={tuple(self.shape)}, nominal {self.dtype}, "
                f"scale {where})")

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        kind = _kind(func, args, kwargs)
        if kind == "product":
            out = _product(func, args, kwargs)
            if out is not None:
                return out
        elif kind == "relayout":
            return cls._wrap(args[0]._codes.transposed(), args[0].dtype)
        elif kind == "alias":
            return cls._wrap(args[0]._codes, args[0].dtype)
        elif kind == "copy":
            c = args[0]._codes
            return cls._wrap(Codes(c.data.clone(), c.scale_inv.clone(), c.axis), args[0].dtype)
        return func(*_plain(args), **_plain(kwargs))


def _plain(tree):
    """The argument tree with every Float8Tensor dequantized to its nominal dtype."""
    return pytree.tree_map(lambda v: v.dequantize() if isinstance(v, Float8Tensor) else v, tree)


def _swaps_2d(func, args):
    """True for t / transpose / permute calls that transpose a 2-D Float8Tensor."""
    x = args[0]
    if not isinstance(x, Float8Tensor) or x.dim() != 2:
        return False
    pk = func.overloadpacket
    if pk is _aten.t:
        return True
    if pk is _aten.transpose:
        return {args[1] % 2, args[2] % 2} == {0, 1}
    if pk is _aten.permute:
        return [d % 2 for d in args[1]] == [1, 0]
    return False


def _kind(func, args, kwargs):
    pk = func.overloadpacket
    if pk in (_aten.mm, _aten.addmm) and "out" not in kwargs:
        return "product"
    if pk in (_aten.t, _aten.transpose, _aten.permute) and _swaps_2d(func, args):
        return "relayout"
    if pk in (_aten.detach, _aten.alias) and isinstance(args[0], Float8Tensor):
        return "alias"
    if pk is _aten.clone and isinstance(args[0], Float8Tensor) and kwargs.get("memory_format") in (
            None, torch.preserve_format, torch.contiguous_format):
        return "copy"
    return "dequantize"


def _operand(x, outer_axis):
    """(data, scale or None, nominal dtype) of a product operand whose non-K axis is ``outer_axis``, or
    None when the library cannot take it as it is (a scale along K, or an unsupported plain dtype)."""
    if isinstance(x, Float8Tensor):
        c = x._codes
        if c.axis is not None and c.axis != outer_axis:
            return None  # the factors vary along K: only dequantization applies them
        return c.data, c.scale_inv, x.dtype
    if x.dtype not in (torch.bfloat16, torch.float32):
        return None
    return x, None, x.dtype


def _product(func, args, kwargs):
    """mm(a, b) or addmm(bias, a, b, beta=1, alpha) on the library, or None to dequantize instead."""
    from . import matmul
    if func.overloadpacket is _aten.mm:
        bias, (a, b), alpha, beta = None, args, 1.0, 1.0
    else:
        bias, a, b = args[:3]
        alpha, beta = kwargs.get("alpha", 1), kwargs.get("beta", 1)
    if beta != 1 or a.dim() != 2 or b.dim() != 2 or a.shape[1] % 16:
        return None
    pa, pb = _operand(a, 0), _operand(b, 1)
    if pa is None or pb is None:
        return None
    if bias is not None:
        if isinstance(bias, Float8Tensor) or bias.dim() != 1 or bias.shape[0] != b.shape[1]:
            return None  # a bias that is not one value per output column
    (da, sa, ta), (db, sb, tb) = pa, pb
    return matmul(da, db, out_dtype=torch.promote_types(ta, tb), bias=bias, alpha=float(alpha), scale_a=sa,
                  scale_b=sb)


def quantize_linear_(module: torch.nn.Module, *, fp8: torch.dtype = torch.float8_e4m3fn, per_row: bool = True,
                     dtype: Optional[torch.dtype] = None) -> torch.nn.Module:
    """Store the weight of every ``nn.Linear`` of ``module`` (in place) as a ``Float8Tensor`` -- one
    scale per output feature by default, E4M3 unless ``fp8`` says otherwise -- so that its forward runs
    the FP8 GEMM.  Layers whose ``in_features`` is not a multiple of 16 (the GEMM's K rule) keep their
    weights.  Inference only.  Returns ``module``."""
    layers = [m for m in module.modules() if isinstance(m, torch.nn.Linear)]
    for layer in layers:
        w = layer.weight
        if isinstance(w, Float8Tensor) or layer.in_features % 16:
            continue
        q = Float8Tensor.from_float(w.data, fp8=fp8, per_row=per_row, dtype=dtype or w.dtype)
        layer.weight = torch.nn.Parameter(q, requires_grad=False)
    return module
