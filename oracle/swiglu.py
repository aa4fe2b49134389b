"""SwiGLU oracle (test infrastructure; see oracle/__init__.py).

Reference: src/picotron/nn/triton_kernels/swiglu.py
  forward  :69 / Triton :26-41   y = silu(g) * u = g * sigmoid(g) * u
  backward :71-81                s = sigmoid(g); dg = dy*u*s*(1 + g*(1 - s)); du = dy*g*s
"""

from __future__ import annotations

import torch
from torch import Tensor


def forward(g: Tensor, u: Tensor, compute: torch.dtype = torch.float64) -> Tensor:
    gc, uc = g.to(compute), u.to(compute)
    return gc * torch.sigmoid(gc) * uc


def backward(dy: Tensor, g: Tensor, u: Tensor, compute: torch.dtype = torch.float64) -> tuple[Tensor, Tensor]:
    d, gc, uc = dy.to(compute), g.to(compute), u.to(compute)
    s = torch.sigmoid(gc)
    dg = d * uc * (s * (1 + gc * (1 - s)))
    du = d * (gc * s)
    return dg, du


def fallback_forward_backward(g: Tensor, u: Tensor, dy: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """The reference's PyTorch path as it runs, in the input dtype (feedforward.py:42 forward,
    swiglu.py:75-81 backward)."""

    y = torch.nn.functional.silu(g) * u
    sigmoid_gate = torch.sigmoid(g)
    silu_gate = g * sigmoid_gate
    silu_derivative = sigmoid_gate * (1 + g * (1 - sigmoid_gate))
    dg = dy * u * silu_derivative
    du = dy * silu_gate
    return y, dg, du
