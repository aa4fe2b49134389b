"""Build ``libpicotron_hip.so`` for gfx950 (MI355X) from ``picotron_amd/csrc``.

Every ``*.hip`` translation unit is compiled by ``hipcc`` in parallel and linked into one
shared library next to this file (in-tree, so it travels with the source tree).  The
build always recompiles; nothing is cached between calls.

Usage: ``python -m picotron_amd.build [-j N] [-v]``.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "libpicotron_hip.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"

OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32 (device pass
# only; the host pass prints a harmless "not a recognized feature" note, filtered below).
COMPILE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

_HOST_FEATURE_NOTE = "'-packed-fp32-ops' is not a recognized feature for this target"


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    for candidate in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if _HOST_FEATURE_NOTE not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1))

    def compile_one(src: Path) -> tuple[Path, str]:
        obj = BUILD_DIR / (src.stem + ".o")
        cmd = [hipcc, *COMPILE_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(src), "-o", str(obj)]
        return obj, _run(cmd)

    objects: list[Path] = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for obj, log in pool.map(compile_one, srcs):
            objects.append(obj)
            if verbose and log.strip():
                print(log, file=sys.stderr)

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def ensure_built() -> Path:
    """The in-tree library, built first when it is not there.  An existing library is used
    as it is: after changing a source, call :func:`build`."""

    if not LIB_PATH.exists():
        build()
    return LIB_PATH


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("-j", "--jobs", type=int, default=None)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args()
    path = build(jobs=args.jobs, verbose=args.verbose)
    print(path)


if __name__ == "__main__":
    main()
