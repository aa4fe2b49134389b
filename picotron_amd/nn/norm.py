"""RMSNorm module with the reference's call surface (src/picotron/models/picotron_decoder.py:20-46).

``RMSNorm(hidden_size, eps=1e-6, *, use_triton_rmsnorm=False)`` holds an fp32 ``weight``
(initialised to ones) and, when the flag is set, runs the fused HIP kernels, warning once
and falling back to the eager formula if they cannot run.  The attribute names
(``use_triton_rmsnorm``, ``_triton_fallback_warned``) are kept because picotron's probes
read them.
"""

from __future__ import annotations

import warnings

import torch
from torch import Tensor, nn

from picotron_amd.nn.triton_kernels.rmsnorm import triton_residual_rms_norm, triton_rms_norm


class RMSNorm(nn.Module):
    """Root mean square normalization with a learned scale."""

    def __init__(
        self, hidden_size: int, eps: float = 1e-6, *, use_triton_rmsnorm: bool = False
    ) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps
        self.use_triton_rmsnorm = use_triton_rmsnorm
        self._triton_fallback_warned = False

    def _warn_fallback(self, error: Exception) -> None:
        if not self._triton_fallback_warned:
            warnings.warn(
                f"Triton RMSNorm unavailable; using PyTorch fallback: {error}",
                RuntimeWarning,
                stacklevel=3,
            )
            self._triton_fallback_warned = True

    def _eager(self, hidden_states: Tensor) -> Tensor:
        variance = hidden_states.pow(2).mean(dim=-1, keepdim=True)
        normalized = hidden_states * torch.rsqrt(variance + self.eps)
        return normalized * self.weight

    def forward(self, hidden_states: Tensor) -> Tensor:
        if self.use_triton_rmsnorm:
            try:
                return triton_rms_norm(hidden_states, self.weight, self.eps)
            except Exception as error:
                self._warn_fallback(error)
        return self._eager(hidden_states)

    def add_and_norm(self, hidden_states: Tensor, residual: Tensor) -> tuple[Tensor, Tensor]:
        """``(h, self(h))`` with ``h = hidden_states + residual``: the decoder block's residual
        add and the norm after it (src/picotron/models/picotron_decoder.py:116-119), fused into
        one kernel on the fast path."""

        if self.use_triton_rmsnorm:
            try:
                return triton_residual_rms_norm(hidden_states, residual, self.weight, self.eps)
            except Exception as error:
                self._warn_fallback(error)
        h = hidden_states + residual
        return h, self._eager(h)
