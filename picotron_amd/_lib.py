"""ctypes binding of ``libpicotron_hip.so`` (C ABI declared in ``include/picotron_hip.h``).

The library is loaded lazily, once per process.  Loading fails loudly with
:class:`HipLibraryUnavailable` (never a silent fallback) when the shared object is missing,
was built for another ABI version, or cannot be opened.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_double, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("PICOTRON_HIP_LIB", Path(__file__).with_name("libpicotron_hip.so")))

ABI_VERSION = 4

PT_FLOAT32 = 0
PT_FLOAT16 = 1
PT_BFLOAT16 = 2

PT_OK = 0
PT_EINVAL = 1
PT_EUNSUPPORTED = 2
PT_ELAUNCH = 3
PT_EDEVICE = 4

_c_int64_p = ctypes.POINTER(c_int64)
_c_float_p = ctypes.POINTER(c_float)

# name -> (restype, argtypes); mirrors include/picotron_hip.h one to one.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "pt_abi_version": (c_int, []),
    "pt_last_error": (ctypes.c_char_p, []),
    "pt_device_supported": (c_int, [c_int]),
    "pt_rmsnorm_fwd": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_float,
         c_int, c_int, c_void_p],
    ),
    "pt_rmsnorm_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int]),
    "pt_rmsnorm_bwd": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
         c_void_p, c_size_t, c_int64, c_int64, c_int, c_int, c_void_p],
    ),
    "pt_rmsnorm_bwd_noalloc": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
         c_int64, c_int64, c_int, c_int, c_void_p],
    ),
    "pt_residual_rmsnorm_fwd": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
         c_void_p, c_int64, c_int64, c_float, c_int, c_int, c_void_p],
    ),
    "pt_residual_rmsnorm_bwd": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
         c_int64, c_void_p, c_void_p, c_size_t, c_int64, c_int64, c_int, c_int, c_void_p],
    ),
    "pt_swiglu_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "pt_swiglu_bwd": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]
    ),
    "pt_rope": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
         c_int64, c_int, c_int, c_int, c_void_p],
    ),
    "pt_cross_entropy_workspace_bytes": (c_size_t, [c_int64]),
    "pt_cross_entropy": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64,
         c_int64, c_void_p, c_int, c_void_p, c_int64, c_int64, c_void_p, c_size_t, c_int,
         c_void_p],
    ),
    "pt_cross_entropy_status": (c_void_p, [c_void_p]),
    "pt_cross_entropy_scale_grad": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64,
         c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int, c_void_p],
    ),
    "pt_cross_entropy_shifted": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64,
         c_int64, c_void_p, c_int, c_void_p, c_int64, c_int64, c_void_p, c_size_t, c_int,
         c_void_p],
    ),
    "pt_cross_entropy_shifted_scale_grad": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64,
         c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int, c_void_p],
    ),
    "pt_adamw_block_elems": (c_int64, []),
    "pt_adamw_step": (
        c_int,
        [c_void_p, c_int64, c_int64, c_double, c_double, c_double, c_double, c_double, c_double,
         c_void_p],
    ),
    "pt_clip_grad_norm_workspace_bytes": (c_size_t, [c_int64]),
    "pt_clip_grad_norm": (
        c_int,
        [c_void_p, c_int64, c_int64, c_double, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "pt_adamw_step_scaled": (
        c_int,
        [c_void_p, c_int64, c_int64, c_double, c_double, c_double, c_double, c_double, c_double,
         c_void_p, c_int, c_void_p],
    ),
    "pt_adamw_step_device_step": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_double, c_double, c_double, c_double, c_double,
         c_void_p, c_int, c_void_p],
    ),
    "pt_adamw_step_device_step_guarded": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_double, c_double, c_double, c_double, c_double,
         c_void_p, c_int, c_void_p, c_void_p, c_void_p],
    ),
    "pt_grad_stats_workspace_bytes": (c_size_t, [c_int64]),
    "pt_grad_stats": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_double, c_int, c_void_p, c_void_p, c_void_p,
         c_void_p, c_size_t, c_void_p],
    ),
    "pt_grad_scale": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "pt_copy": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
}


class HipLibraryUnavailable(RuntimeError):
    """The HIP kernel library could not be loaded (missing, stale, or wrong ABI)."""


class HipKernelError(RuntimeError):
    """A library entry point rejected its arguments or failed to launch."""

    def __init__(self, fn: str, code: int, message: str) -> None:
        super().__init__(f"{fn} failed (code {code}): {message}")
        self.fn = fn
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        if _load_error is not None:
            raise HipLibraryUnavailable(_load_error)
        if not LIB_PATH.exists():
            _load_error = (
                f"{LIB_PATH} is not built (run `python -m picotron_amd.build` or "
                "`python -c 'import __graft_entry__ as g; g.build()'`)"
            )
            raise HipLibraryUnavailable(_load_error)
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as error:
            _load_error = f"cannot load {LIB_PATH}: {error}"
            raise HipLibraryUnavailable(_load_error) from error
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                _load_error = f"{LIB_PATH} lacks symbol {name}; rebuild it"
                raise HipLibraryUnavailable(_load_error)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.pt_abi_version()
        if version != ABI_VERSION:
            _load_error = f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
            raise HipLibraryUnavailable(_load_error)
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises :class:`HipLibraryUnavailable` if it cannot be loaded."""

    return _lib if _lib is not None else _load()


def is_available() -> bool:
    try:
        lib()
    except HipLibraryUnavailable:
        return False
    return True


def unavailable_reason() -> str | None:
    try:
        lib()
    except HipLibraryUnavailable as error:
        return str(error)
    return None


def check(fn: str, rc: int) -> None:
    """Raise :class:`HipKernelError` with the library's message for a nonzero return."""

    if rc != PT_OK:
        message = lib().pt_last_error()
        raise HipKernelError(fn, rc, message.decode() if message else "")


_bound: dict[str, object] = {}


def call(fn: str, *args) -> None:
    """Call entry point ``fn`` and raise :class:`HipKernelError` on a nonzero return (the bound
    function object is looked up once per name)."""

    f = _bound.get(fn)
    if f is None:
        f = _bound[fn] = getattr(lib(), fn)
    rc = f(*args)
    if rc != PT_OK:
        check(fn, rc)
