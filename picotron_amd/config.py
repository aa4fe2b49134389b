"""``model.triton_kernels`` flags (reference src/picotron/config/config.py:72-92).

Same names, strict-bool validation and defaults (all False).  ``rmsnorm``, ``swiglu``,
``rope``, ``cross_entropy`` and ``adamw`` select the HIP kernels of this package;
``attention`` is accepted and always falls back (fused attention is not part of it).
"""

from __future__ import annotations

from dataclasses import dataclass

FLAG_NAMES = ("rmsnorm", "swiglu", "rope", "attention", "cross_entropy", "adamw")


class ConfigValidationError(ValueError):
    """Raised when a kernel-flag configuration is invalid."""


def _require_bool(name: str, value: object) -> None:
    if not isinstance(value, bool):
        raise ConfigValidationError(f"'{name}' must be a boolean; got {value!r}.")


@dataclass(frozen=True, slots=True)
class TritonKernelsConfig:
    """Explicit opt-ins for the optional fused kernels."""

    rmsnorm: bool = False
    swiglu: bool = False
    rope: bool = False
    attention: bool = False
    cross_entropy: bool = False
    adamw: bool = False

    def __post_init__(self) -> None:
        for field_name in FLAG_NAMES:
            _require_bool(field_name, getattr(self, field_name))

    @classmethod
    def from_mapping(cls, values: dict) -> "TritonKernelsConfig":
        """Build from a YAML mapping; unknown keys are errors (as the reference loader)."""

        unknown = set(values) - set(FLAG_NAMES)
        if unknown:
            raise ConfigValidationError(f"unknown triton_kernels keys: {sorted(unknown)}")
        return cls(**values)
