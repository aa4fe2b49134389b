"""AdamW oracle (test infrastructure; see oracle/__init__.py).

Reference: src/picotron/nn/triton_kernels/adamw.py:34-47 falls back to optimizer.step() of
torch.optim.AdamW(params, lr, betas, eps, weight_decay) (train_loop.py:308-325), i.e.
torch's single-tensor Adam with decoupled weight decay, amsgrad=False:
  p *= 1 - lr*wd; m = lerp(m, g, 1-b1); v = v*b2 + (1-b2)*g*g;
  p -= (lr / (1 - b1^t)) * m / (sqrt(v) / sqrt(1 - b2^t) + eps)
"""

from __future__ import annotations

import torch
from torch import Tensor


def step(
    p: Tensor,
    g: Tensor,
    m: Tensor,
    v: Tensor,
    *,
    t: int,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    compute: torch.dtype = torch.float64,
) -> tuple[Tensor, Tensor, Tensor]:
    """One step from state (m, v) at step t-1 to step t; returns new (p, m, v) in compute."""

    pc, gc, mc, vc = (x.to(compute) for x in (p, g, m, v))
    pc = pc * (1 - lr * weight_decay)
    mc = mc + (1 - beta1) * (gc - mc)
    vc = vc * beta2 + (1 - beta2) * gc * gc
    bc1 = 1 - beta1**t
    bc2 = 1 - beta2**t
    denom = torch.sqrt(vc) / (bc2**0.5) + eps
    pc = pc - (lr / bc1) * mc / denom
    return pc, mc, vc


def fallback_step(optimizer: torch.optim.Optimizer) -> None:
    """The reference's fallback as it runs: torch's own AdamW step."""

    optimizer.step()


def clip_grad_norm(grads: list[Tensor], max_norm: float, compute: torch.dtype = torch.float64) -> tuple[Tensor, list[Tensor]]:
    """torch.nn.utils.clip_grad_norm_ with norm_type 2, as the train loop calls it before
    the step (reference src/picotron/training/train_loop.py:338-350): total = ||all grads||_2,
    coef = min(max_norm / (total + 1e-6), 1), every gradient multiplied by coef.  Returns
    (total, clipped grads) in ``compute``."""

    gs = [g.to(compute) for g in grads]
    if not gs:
        return torch.zeros((), dtype=compute), []
    total = torch.sqrt(sum((g * g).sum() for g in gs))
    coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    return total, [g * coef for g in gs]


def unscale_and_check(grads: list[Tensor], scale: float) -> tuple[bool, list[Tensor]]:
    """The ZeRO optimizer's unscale_and_check_ (reference src/picotron/parallel/zero.py:139-163)
    on one rank: (True, grads unchanged) if any gradient holds inf or NaN, else
    (False, every gradient multiplied by the Python float 1/scale in its own dtype)."""

    if any(not bool(torch.isfinite(g).all()) for g in grads):
        return True, list(grads)
    inverse_scale = 1.0 / scale
    return False, [g * inverse_scale for g in grads]


def zero_clip_grad_norm(grads: list[Tensor], max_norm: float, compute: torch.dtype = torch.float64) -> tuple[Tensor, list[Tensor]]:
    """The ZeRO optimizer's clip_grad_norm_ (reference src/picotron/parallel/zero.py:165-186)
    on one rank: total = ||all grads||_2, coef = max_norm / (total + 1e-6), gradients
    multiplied by coef only when coef < 1.  Returns (total, grads) in ``compute``."""

    gs = [g.to(compute) for g in grads]
    if not gs:
        return torch.zeros((), dtype=compute), []
    total = torch.sqrt(sum((g * g).sum() for g in gs))
    coef = max_norm / (total + 1e-6)
    if bool(coef < 1):
        gs = [g * coef for g in gs]
    return total, gs
