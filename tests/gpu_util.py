"""Helpers shared by the GPU parity tests (tolerances, seeded device tensors)."""

from __future__ import annotations

import numpy as np
import torch

# Tolerances: fp32 against the reference's PyTorch fallback at 1e-5 relative (with an
# absolute floor of 1e-6 of the tensor's scale, for entries that cancel to ~0); bf16 and
# fp16 against an fp32/fp64 oracle.
BF16 = dict(atol=2e-2, rtol=1.6e-2)
FP16 = dict(atol=2e-3, rtol=2e-3)


def close_fp32(
    actual: torch.Tensor, expected: torch.Tensor, rtol: float = 1e-5, scale: float | None = None
) -> None:
    """|a - e| <= rtol*|e| + 1e-6*scale.  ``scale`` defaults to max|e|; pass the magnitude of
    the summands when the result is a near-cancelling difference of them."""

    expected = expected.detach().to(actual.device)
    if scale is None:
        scale = float(expected.abs().max()) if expected.numel() else 0.0
    torch.testing.assert_close(
        actual.double(), expected.double(), rtol=rtol, atol=max(1e-6 * scale, 1e-12)
    )


def close(
    actual: torch.Tensor, expected: torch.Tensor, dtype: torch.dtype, scale: float | None = None
) -> None:
    expected = expected.detach().to(actual.device)
    if dtype == torch.float32:
        close_fp32(actual, expected, scale=scale)
    elif dtype == torch.bfloat16:
        torch.testing.assert_close(actual.double(), expected.double(), **BF16)
    else:
        torch.testing.assert_close(actual.double(), expected.double(), **FP16)


def randn(shape, dtype, device, seed, scale=1.0, shift=0.0):
    """Seeded N(shift, scale^2) generated in fp32 on ``device``, then cast."""

    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * scale + shift).to(dtype)


def from_npz(array: np.ndarray, device, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(array)).to(device)
    return t if dtype is None else t.to(dtype)
