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

from picotron_amd.nn.triton_kernels.rmsnorm import triton_rms_norm


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

    def forward(self, hidden_states: Tensor) -> Tensor:
        if self.use_triton_rmsnorm:
            try:
                return triton_rms_norm(hidden_states, self.weight, self.eps)
            except Exception as error:
                if not self._triton_fallback_warned:
                    warnings.warn(
                        f"Triton RMSNorm unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._triton_fallback_warned = True
        variance = hidden_states.pow(2).mean(dim=-1, keepdim=True)
        normalized = hidden_states * torch.rsqrt(variance + self.eps)
        return normalized * self.weight
