"""Capability report for the fused kernels (reference src/picotron/utils/hardware.py:31-38,
93-108).

``detect_triton_support(enabled=..., device=...)`` keeps the reference's name and
``TritonReport`` fields: ``installed`` means the HIP kernel library loads,
``hardware_compatible`` means the device is a gfx950 GPU, and ``available`` requires both
plus ``enabled``.  Never enables anything implicitly.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from picotron_amd import _lib


@dataclass(frozen=True, slots=True)
class TritonReport:
    """Optional fused-kernel status; disabled unless explicitly requested."""

    enabled: bool
    installed: bool
    hardware_compatible: bool
    available: bool


def detect_triton_support(
    *, enabled: bool = False, device: int | torch.device | None = None
) -> TritonReport:
    """Report fused-kernel status without enabling it implicitly."""

    installed = _lib.is_available()
    hardware_compatible = False
    if installed and torch.cuda.is_available():
        if isinstance(device, torch.device):
            index = device.index if device.index is not None else torch.cuda.current_device()
        elif device is None:
            index = torch.cuda.current_device()
        else:
            index = int(device)
        hardware_compatible = bool(_lib.lib().pt_device_supported(index))
    return TritonReport(
        enabled=enabled,
        installed=installed,
        hardware_compatible=hardware_compatible,
        available=enabled and installed and hardware_compatible,
    )
