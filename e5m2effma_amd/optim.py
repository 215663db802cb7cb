"""``AdamW``: a ``torch.optim`` optimizer whose update is the fused ``e5ma_adam`` kernel.

Same hyper-parameters and update as ``torch.optim.AdamW`` (or Adam, ``adamw=False``), like the reference
package's optimizer (reference ``binds/python/e5m2effma/optim.py:9-53``): one kernel launch per
parameter reads p, g, m, v once and writes p, m, v in place.  FP32 or BF16 parameters; FP32 / BF16 /
FP16 gradients; moments in ``state_dtype`` (FP32 by default, BF16 halves the optimizer memory).

Beyond the reference: ``grad_scale`` (per group) multiplies the gradient inside the kernel, e.g. to
undo a loss scale, and ``fp8_copy=torch.float8_e5m2 / float8_e4m3fn`` keeps an FP8 copy of every
parameter, written by the same launch, with delayed scaling: each step quantizes with
``scale = margin * max_finite / amax`` of the previous step's weights (amax recorded by the kernel), so
``state["param_fp8"]`` and ``state["fp8_scale_inv"]`` always describe the current weights.
"""
from typing import Iterable, Optional, Tuple

import torch

__all__ = ["AdamW"]

_STATE_DTYPES = (torch.float32, torch.bfloat16)
_QMAX = {torch.float8_e5m2: 57344.0, torch.float8_e4m3fn: 448.0}


def _validate(lr, betas, eps, weight_decay, grad_scale):
    if not (lr >= 0.0 and eps >= 0.0 and weight_decay >= 0.0):
        raise ValueError(f"AdamW needs lr, eps and weight_decay >= 0; got lr={lr}, eps={eps}, "
                         f"weight_decay={weight_decay}")
    if len(betas) != 2 or not all(0.0 <= b < 1.0 for b in betas):
        raise ValueError(f"AdamW betas must be two values in [0, 1), got {tuple(betas)}")
    if not grad_scale > 0.0:
        raise ValueError(f"AdamW grad_scale must be positive, got {grad_scale}")


class AdamW(torch.optim.Optimizer):
    """AdamW / Adam on the fused kernel.

    ``AdamW(params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, *, adamw=True,
    state_dtype=None, grad_scale=1.0, fp8_copy=None, fp8_margin=1.0)``.  Parameters must be contiguous
    tensors on a gfx950 device.  State per parameter: ``step`` (int), ``exp_avg``, ``exp_avg_sq``, and with
    ``fp8_copy`` also ``param_fp8``, ``fp8_scale`` (1 float), ``fp8_scale_inv`` (1 float) and ``fp8_amax``.
    """

    def __init__(self, params: Iterable, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 1e-2, *, adamw: bool = True,
                 state_dtype: Optional[torch.dtype] = None, grad_scale: float = 1.0,
                 fp8_copy: Optional[torch.dtype] = None, fp8_margin: float = 1.0):
        _validate(lr, betas, eps, weight_decay, grad_scale)
        if state_dtype is not None and state_dtype not in _STATE_DTYPES:
            raise TypeError(f"AdamW state_dtype must be torch.float32 or torch.bfloat16, got {state_dtype}")
        if fp8_copy is not None and fp8_copy not in _QMAX:
            raise TypeError(f"AdamW fp8_copy must be torch.float8_e5m2 or torch.float8_e4m3fn, got {fp8_copy}")
        if not fp8_margin > 0.0:
            raise ValueError(f"AdamW fp8_margin must be positive, got {fp8_margin}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay,
                                      adamw=adamw, state_dtype=state_dtype or torch.float32,
                                      grad_scale=grad_scale, fp8_copy=fp8_copy, fp8_margin=fp8_margin))

    def _init_state(self, p, group):
        st = self.state[p]
        st["step"] = 0
        st["exp_avg"] = torch.zeros(p.shape, dtype=group["state_dtype"], device=p.device)
        st["exp_avg_sq"] = torch.zeros(p.shape, dtype=group["state_dtype"], device=p.device)
        fmt = group["fp8_copy"]
        if fmt is not None:
            # the first copy is quantized with the current weights' own amax
            amax = p.detach().abs().amax().float().clamp_min(1e-12).reshape(1)
            st["param_fp8"] = torch.empty(p.shape, dtype=fmt, device=p.device)
            st["fp8_scale"] = amax.reciprocal() * (group["fp8_margin"] * _QMAX[fmt])
            st["fp8_scale_inv"] = 1.0 / st["fp8_scale"]
            st["fp8_amax"] = torch.zeros(1, dtype=torch.float32, device=p.device)
        return st

    def _launches(self):
        """(parameter, its gradient, its state, its group) for every parameter with a gradient."""
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise ValueError("AdamW takes dense gradients; this parameter's gradient is sparse")
                st = self.state[p] or self._init_state(p, group)
                yield p, p.grad, st, group

    @torch.no_grad()
    def step(self, closure=None):
        """One update of every parameter that has a gradient; returns the closure's loss (if given)."""
        from . import adam_step
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for p, g, st, group in self._launches():
            st["step"] += 1
            fp8 = group["fp8_copy"] is not None
            if fp8 and st["step"] > 1:
                # delayed scaling: this step's copy uses the amax of the weights the previous step wrote
                amax = st["fp8_amax"].clamp_min(1e-12)
                torch.mul(amax.reciprocal(), group["fp8_margin"] * _QMAX[group["fp8_copy"]], out=st["fp8_scale"])
                st["fp8_amax"].zero_()
            adam_step(p, g, st["exp_avg"], st["exp_avg_sq"], lr=group["lr"], betas=group["betas"],
                      eps=group["eps"], weight_decay=group["weight_decay"], step=st["step"],
                      adamw=group["adamw"], grad_scale=group["grad_scale"],
                      param_fp8=st["param_fp8"] if fp8 else None, fp8_scale=st["fp8_scale"] if fp8 else None,
                      fp8_amax=st["fp8_amax"] if fp8 else None)
            if fp8:
                torch.reciprocal(st["fp8_scale"], out=st["fp8_scale_inv"])
        return loss
