"""``AdamW``: a ``torch.optim`` optimizer whose step is the fused ``e5ma_adam`` kernel.

Interface of the reference's ``binds/python/e5m2effma/optim.py:9-53``: the hyper-parameters and semantics of
``torch.optim.AdamW`` (``adamw=False`` gives Adam with L2 weight decay), float32 / bfloat16 parameters,
float32 / bfloat16 / float16 gradients, and ``state_dtype`` for the two moments (float32 by default;
bfloat16 halves the optimizer state).  One kernel launch per parameter tensor, on torch's current stream.
"""
from typing import Iterable, Optional, Tuple

import torch

_STATE_DTYPES = (torch.float32, torch.bfloat16)


class AdamW(torch.optim.Optimizer):
    def __init__(self, params: Iterable, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 1e-2, *, adamw: bool = True,
                 state_dtype: Optional[torch.dtype] = None):
        if min(lr, eps, weight_decay) < 0.0:
            raise ValueError(f"lr, eps and weight_decay must be non-negative (got {lr}, {eps}, {weight_decay})")
        if not all(0.0 <= b < 1.0 for b in betas):
            raise ValueError(f"betas must be in [0, 1), got {tuple(betas)}")
        if state_dtype is not None and state_dtype not in _STATE_DTYPES:
            raise TypeError(f"state_dtype must be torch.float32 or torch.bfloat16, got {state_dtype}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay, adamw=adamw,
                                      state_dtype=state_dtype or torch.float32))

    def _state_of(self, p, group):
        st = self.state[p]
        if not st:
            st["step"] = 0
            for name in ("exp_avg", "exp_avg_sq"):
                st[name] = torch.zeros(p.shape, dtype=group["state_dtype"], device=p.device)
        return st

    @torch.no_grad()
    def step(self, closure=None):
        from . import adam_step
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise ValueError("AdamW does not support sparse gradients")
                st = self._state_of(p, group)
                st["step"] += 1
                adam_step(p, p.grad, st["exp_avg"], st["exp_avg_sq"], lr=group["lr"], betas=group["betas"],
                          eps=group["eps"], weight_decay=group["weight_decay"], step=st["step"],
                          adamw=group["adamw"])
        return loss
