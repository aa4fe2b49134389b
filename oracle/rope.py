"""RoPE oracle (test infrastructure; see oracle/__init__.py).

Reference: src/picotron/nn/rope.py
  rotary_cos_sin          :13-32  inv = 1/theta^(arange(0, D, 2)/D) (fp32); angle = outer(pos, inv)
  apply_rotary_embedding  :35-51  interleaved pairs (2i, 2i+1): (a, b) -> (a c - b s, a s + b c)
The rotate-half layout (pairs (i, i + D/2)) has no reference code; it is the same rotation
on a permuted head dimension: rotate_half(P x) = P interleaved(x), P = [evens, odds].
"""

from __future__ import annotations

import torch
from torch import Tensor


def tables(seq: int, head_dim: int, theta: float, device=None) -> tuple[Tensor, Tensor]:
    """fp32 (cos, sin) [seq, head_dim/2], the reference formula evaluated in fp32."""

    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    pos = torch.arange(seq, device=device, dtype=torch.float32)
    ang = torch.outer(pos, inv)
    return ang.cos(), ang.sin()


def rotate(
    x: Tensor,
    cos: Tensor,
    sin: Tensor,
    layout: str = "interleaved",
    inverse: bool = False,
    compute: torch.dtype = torch.float64,
) -> Tensor:
    """Rotate (..., seq, head_dim) states; ``inverse`` rotates by -angle (the backward)."""

    xc = x.to(compute)
    seq = x.size(-2)
    c = cos[:seq].to(compute)
    s = sin[:seq].to(compute)
    if inverse:
        s = -s
    if layout == "interleaved":
        a, b = xc[..., 0::2], xc[..., 1::2]
        out = torch.stack((a * c - b * s, a * s + b * c), dim=-1)
        return out.flatten(start_dim=-2)
    if layout == "rotate_half":
        half = x.size(-1) // 2
        a, b = xc[..., :half], xc[..., half:]
        return torch.cat((a * c - b * s, a * s + b * c), dim=-1)
    raise ValueError(f"unknown layout {layout!r}")


def fallback_forward_backward(
    x: Tensor, cos: Tensor, sin: Tensor, dy: Tensor
) -> tuple[Tensor, Tensor]:
    """The reference's eager path as it runs (apply_rotary_embedding + autograd), in the
    input dtype: returns (y, dx)."""

    xr = x.detach().requires_grad_(True)
    c = cos.unsqueeze(0).unsqueeze(0)
    s = sin.unsqueeze(0).unsqueeze(0)
    even, odd = xr[..., 0::2], xr[..., 1::2]
    y = torch.stack((even * c - odd * s, even * s + odd * c), dim=-1).flatten(start_dim=-2)
    y.backward(dy)
    return y.detach(), xr.grad
