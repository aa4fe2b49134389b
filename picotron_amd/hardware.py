"""Capability report for the fused kernels (reference src/picotron/utils/hardware.py:31-38,
93-108).

``detect_triton_support(enabled=..., device=...)`` keeps the reference's name and
``TritonReport`` fields: ``installed`` means the HIP kernel library loads,
``hardware_compatible`` means the device is a gfx950 GPU, and ``available`` requires both
plus ``enabled``.  Never enables anything implicitly.

``kernel_status_rows(flags)`` gives the two kernel rows of the run banner
(src/picotron/logging/display.py:315-338) from the live state rather than the reference's
fixed "rmsnorm=real swiglu=real rope=fallback ..." string.
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


# Kernels of the run banner, in its order; attention has no fused kernel here.
_BANNER_KERNELS = ("rmsnorm", "swiglu", "rope", "attention", "cross_entropy", "adamw")


def kernel_status_rows(
    flags, *, device: int | torch.device | None = None
) -> tuple[tuple[str, str], tuple[str, str]]:
    """The banner's ``("Triton kernels", ...)`` and ``("Triton status", ...)`` rows for a
    ``TritonKernelsConfig`` (display.py:315-338): "off" when no flag is set, "active: ..."
    when the enabled kernels run on the HIP library, "requested; fallback: ..." when they
    cannot; the status row says per kernel whether the HIP kernel ("real") or the PyTorch
    fallback would run."""

    enabled = tuple(name for name in _BANNER_KERNELS if getattr(flags, name))
    report = detect_triton_support(enabled=bool(enabled), device=device)
    if not enabled:
        kernels = "off"
    elif report.available:
        kernels = "active: " + ", ".join(enabled)
    else:
        kernels = "requested; fallback: " + ", ".join(enabled)
    runs = report.installed and report.hardware_compatible
    status = " ".join(
        f"{name}={'real' if runs and name != 'attention' else 'fallback'}"
        for name in _BANNER_KERNELS
    )
    return ("Triton kernels", kernels), ("Triton status", status)
