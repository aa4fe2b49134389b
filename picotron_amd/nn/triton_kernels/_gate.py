"""Shared launch gate for the fused kernels: library loaded, GPU tensors, gfx950 device.

Replaces the Triton checks of the reference (``_TRITON_AVAILABLE``, ``is_cuda``,
``get_device_capability(...)[0] >= 7``; e.g. src/picotron/nn/triton_kernels/rmsnorm.py:140-145).
Each op passes its own ``*Unavailable`` exception type, so callers keep catching what the
reference raised.
"""

from __future__ import annotations

import os

import torch
from torch import Tensor

from picotron_amd import _lib, ops

# PICOTRON_HIP_DISABLE=1 makes every fused op report itself unavailable (forces the
# PyTorch fallbacks, e.g. to compare against them on a GPU host).
_DISABLED_ENV = "PICOTRON_HIP_DISABLE"


# The process-wide parts of the gate are constants to torch.compile: it evaluates them once
# while tracing and keeps the answer, so a compiled model neither re-checks them per call nor
# breaks its graph at the ctypes and environment lookups.


@torch.compiler.assume_constant_result
def _process_reason() -> str:
    """'' if the fused kernels may run in this process, else why not ('{op}' is a placeholder)."""

    if os.environ.get(_DISABLED_ENV, "") not in ("", "0"):
        return "HIP {op} disabled by " + _DISABLED_ENV + "."
    reason = _lib.unavailable_reason()
    return "" if reason is None else "HIP kernel library unavailable: " + reason


@torch.compiler.assume_constant_result
def _device_supported(index: int) -> bool:
    return ops.device_supported(index)


def require_hip(exc: type[RuntimeError], op: str, *tensors: Tensor) -> None:
    reason = _process_reason()
    if reason:
        raise exc(reason.replace("{op}", op))
    for t in tensors:
        if not t.is_cuda:
            raise exc(f"HIP {op} requires GPU tensors.")
    index = tensors[0].device.index
    if index is None:
        index = torch.cuda.current_device()
    if not _device_supported(index):
        raise exc(f"HIP {op} requires a gfx950 (MI355X) device.")
