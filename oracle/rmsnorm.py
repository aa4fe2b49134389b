"""RMSNorm oracle (test infrastructure; see oracle/__init__.py).

Reference: src/picotron/nn/triton_kernels/rmsnorm.py
  _inverse_rms       :49-53   r = rsqrt(mean(x.float()^2) + eps)
  _pytorch_forward   :56-60   y = (x.float() * r * w.float()).to(x.dtype)
  backward           :110-134 wg = g*w; dm = mean(wg*x); dx = r*(wg - x*r^2*dm);
                              dW = sum_rows(g*x*r)
"""

from __future__ import annotations

import torch
from torch import Tensor


def forward(x: Tensor, w: Tensor, eps: float, compute: torch.dtype = torch.float64) -> tuple[Tensor, Tensor]:
    """(y, rstd) in ``compute``; rstd has shape x.shape[:-1]."""

    xc = x.to(compute)
    ms = (xc * xc).mean(dim=-1)
    rstd = 1.0 / torch.sqrt(ms + eps)
    y = xc * rstd.unsqueeze(-1) * w.to(compute)
    return y, rstd


def backward(
    dy: Tensor, x: Tensor, w: Tensor, eps: float, compute: torch.dtype = torch.float64
) -> tuple[Tensor, Tensor]:
    """(dx, dW) in ``compute`` for upstream gradient ``dy``."""

    xc, wc, gc = x.to(compute), w.to(compute), dy.to(compute)
    _, rstd = forward(x, w, eps, compute)
    r = rstd.unsqueeze(-1)
    wg = gc * wc
    dm = (wg * xc).mean(dim=-1, keepdim=True)
    dx = r * (wg - xc * (r * r) * dm)
    dw = (gc * xc * r).reshape(-1, w.numel()).sum(dim=0)
    return dx, dw


def fallback_forward_backward(
    x: Tensor, w: Tensor, eps: float, dy: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The reference's PyTorch path as it runs (custom Function with the PyTorch forward):
    returns (y, rstd, dx, dW) in the reference's output dtypes."""

    xf = x.float()
    inverse_rms = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    y = (xf * inverse_rms * w.float()).to(dtype=x.dtype)
    g = dy.float()
    wf = w.float()
    weighted_grad = g * wf
    dot_mean = (weighted_grad * xf).mean(dim=-1, keepdim=True)
    dx = inverse_rms * (weighted_grad - xf * inverse_rms.square() * dot_mean)
    dw = (g * xf * inverse_rms).reshape(-1, w.numel()).sum(dim=0)
    return y, inverse_rms.squeeze(-1), dx.to(x.dtype), dw.to(w.dtype)


def residual_forward(
    x: Tensor, residual: Tensor, w: Tensor, eps: float, compute: torch.dtype = torch.float64
) -> tuple[Tensor, Tensor, Tensor]:
    """The decoder block's residual add and the norm after it (reference
    src/picotron/models/picotron_decoder.py:116-119): h = x + residual as stored in x's dtype
    (torch adds in fp32 and rounds once), then (y, rstd) of the norm of that stored h.
    Returns (h in x's dtype, y in compute, rstd in compute)."""

    h = (x.float() + residual.float()).to(x.dtype) if x.dtype != torch.float64 else x + residual
    y, rstd = forward(h, w, eps, compute)
    return h, y, rstd


def residual_backward(
    dy: Tensor, dh_in: Tensor | None, h: Tensor, w: Tensor, eps: float, compute: torch.dtype = torch.float64
) -> tuple[Tensor, Tensor]:
    """(dh, dW): dh = the norm's input gradient + dh_in (the gradient reaching h from the
    block's final residual add); dh is also the gradient of x and of residual."""

    dx, dw = backward(dy, h, w, eps, compute)
    if dh_in is not None:
        dx = dx + dh_in.to(compute)
    return dx, dw
