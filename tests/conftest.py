"""Test configuration: repo root on sys.path, the ``gpu`` marker, shared helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_sessionstart(session: pytest.Session) -> None:
    """Build the in-tree library once if it is missing (a fresh checkout); an existing one,
    or one named by PICOTRON_HIP_LIB, is used as it is."""

    if "PICOTRON_HIP_LIB" not in os.environ:
        from picotron_amd.build import ensure_built

        ensure_built()


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library"
    )


@pytest.fixture(scope="session")
def gpu():
    """The GPU device for HIP parity tests; fails (not skips) if the library is missing."""

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from picotron_amd import _lib, ops

    _lib.lib()  # raises HipLibraryUnavailable loudly if the .so is missing
    if not ops.device_supported(0):
        pytest.fail("GPU 0 is not a gfx950 device")
    return torch.device("cuda:0")
