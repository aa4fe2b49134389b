"""The C-ABI library loads, exports every entry point include/picotron_hip.h declares, and
its host-side queries and argument validation behave.  No kernel launches (CPU only)."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT
from picotron_amd import _lib

HEADER = ROOT / "include" / "picotron_hip.h"


# An 8-byte-aligned host record, so that validation reaches the step-table check (nothing is
# launched: the entry point rejects the missing step table first).
_HOST_TABLE = (ctypes.c_int64 * 6)()


def _declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(pt_[a-z0-9_]+)\s*\(", text))


def test_library_loads_with_matching_abi_version():
    lib = _lib.lib()
    assert lib.pt_abi_version() == _lib.ABI_VERSION
    header_version = re.search(r"#define PT_ABI_VERSION (\d+)", HEADER.read_text()).group(1)
    assert int(header_version) == _lib.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared_functions()
    assert len(declared) >= 16
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in sorted(declared):
        assert hasattr(raw, name), f"{name} declared in the header but not exported"
    assert declared == set(_lib.SIGNATURES), "ctypes signature table differs from the header"


def test_header_constants_match_binding():
    text = HEADER.read_text()
    for name in ("PT_FLOAT32", "PT_FLOAT16", "PT_BFLOAT16", "PT_OK", "PT_EINVAL",
                 "PT_EUNSUPPORTED", "PT_ELAUNCH", "PT_EDEVICE"):
        value = int(re.search(rf"#define {name} (\d+)", text).group(1))
        assert getattr(_lib, name) == value


def test_workspace_queries():
    lib = _lib.lib()
    # RMSNorm backward at 16384 x 4096: 512 partial rows of 4096 fp32
    assert lib.pt_rmsnorm_bwd_workspace_bytes(16384, 4096, _lib.PT_BFLOAT16) == 512 * 4096 * 4
    # 3 rows: the element-wise path (2 rows per 8-wave block) needs 2 partial rows
    assert lib.pt_rmsnorm_bwd_workspace_bytes(3, 128, _lib.PT_FLOAT32) == 2 * 128 * 4
    assert lib.pt_rmsnorm_bwd_workspace_bytes(0, 128, _lib.PT_FLOAT32) == 0
    assert lib.pt_cross_entropy_workspace_bytes(8192) == 16 + 8192 * 8  # row losses + row lse
    assert lib.pt_adamw_block_elems() == 1024


@pytest.mark.parametrize(
    "fn,args,code",
    [
        ("pt_rmsnorm_fwd", (None, 0, None, None, 0, None, 4, 8, 1e-6, 0, 0, None), _lib.PT_EINVAL),
        ("pt_rmsnorm_fwd", (None, 0, None, None, 0, None, 4, 8, 1e-6, 7, 0, None), _lib.PT_EINVAL),
        ("pt_rmsnorm_fwd", (None, 0, None, None, 0, None, 4, 1 << 22, 1e-6, 0, 0, None), _lib.PT_EUNSUPPORTED),
        ("pt_swiglu_fwd", (None, None, None, -1, 2, None), _lib.PT_EINVAL),
        ("pt_rope", (None, None, None, None, None, None, 7, None, None, 1, 0, 0, 2, None), _lib.PT_EINVAL),
        ("pt_adamw_step", (None, 1, 1, 1e-3, 0.9, 0.99, 1e-8, 0.0, 1.0, None), _lib.PT_EINVAL),
        ("pt_adamw_step_device_step", (None, 1, 1, None, 1e-3, 0.9, 0.99, 1e-8, 0.0, None, 0, None), _lib.PT_EINVAL),
        ("pt_adamw_step_device_step", (ctypes.addressof(_HOST_TABLE), 1, 1, None, 1e-3, 0.9, 0.99, 1e-8, 0.0, None, 0, None), _lib.PT_EINVAL),
        # the guarded step: a step table, and grad_scale, found_inf and inv_scale, are required
        ("pt_adamw_step_device_step_guarded", (ctypes.addressof(_HOST_TABLE), 1, 1, None, 1e-3, 0.9, 0.99, 1e-8, 0.0, 16, 1, 16, 16, None), _lib.PT_EINVAL),
        ("pt_adamw_step_device_step_guarded", (ctypes.addressof(_HOST_TABLE), 1, 1, ctypes.addressof(_HOST_TABLE), 1e-3, 0.9, 0.99, 1e-8, 0.0, 16, 1, None, 16, None), _lib.PT_EINVAL),
        ("pt_adamw_step_device_step_guarded", (ctypes.addressof(_HOST_TABLE), 1, 1, ctypes.addressof(_HOST_TABLE), 1e-3, 0.9, 0.99, 1e-8, 0.0, None, 1, 16, 16, None), _lib.PT_EINVAL),
        # more records than blocks: a record without a block (an empty tensor) is refused
        ("pt_adamw_step", (ctypes.addressof(_HOST_TABLE), 2, 1, 1e-3, 0.9, 0.99, 1e-8, 0.0, 1.0, None), _lib.PT_EINVAL),
        ("pt_grad_scale", (ctypes.addressof(_HOST_TABLE), 3, 2, None, None), _lib.PT_EINVAL),
        ("pt_copy", (None, None, 16, None), _lib.PT_EINVAL),
        ("pt_cross_entropy", (None, 4, 1, 8, 0, 8, None, 1, 0, -100, None, 0, None, 0, 0, None, 0, 7, None), _lib.PT_EINVAL),
        ("pt_cross_entropy_shifted", (None, 2, 3, 24, 8, 8, None, 3, 1, -100, None, 0, None, 0, 0, None, 0, 2, None), _lib.PT_EINVAL),
        ("pt_cross_entropy_shifted", (None, 2, 3, 24, 8, 1 << 31, None, 3, 1, -100, None, 0, None, 0, 0, None, 0, 2, None), _lib.PT_EUNSUPPORTED),
        ("pt_cross_entropy_shifted_scale_grad", (None, 2, 3, 24, 8, 8, None, 3, 1, -100, None, None, 0, 0, None, 2, None), _lib.PT_EINVAL),
        # fp16 needs the forward's workspace (n_valid): checked before anything is read
        ("pt_cross_entropy_scale_grad", (16, 4, 1, 8, 0, 8, 16, 1, 0, -100, 16, None, 0, 0, None, 1, None), _lib.PT_EINVAL),
        # a separate gradient whose rows start in another 16-byte phase than the logits rows
        # (the addresses are never dereferenced: the check comes before any launch)
        ("pt_cross_entropy", (4096, 4, 1, 8, 0, 8, 8192, 1, 0, -100, 12288, 1, 4098, 8, 0, 16384, 1 << 20, 2, None), _lib.PT_EINVAL),
        ("pt_cross_entropy", (4096, 4, 1, 8, 0, 8, 8192, 1, 0, -100, 12288, 1, 4096 + 64, 9, 0, 16384, 1 << 20, 2, None), _lib.PT_EINVAL),
        ("pt_cross_entropy_shifted_scale_grad", (4096, 2, 3, 24, 8, 8, 8192, 3, 1, -100, 12288, 4100, 24, 8, 16384, 1, None), _lib.PT_EINVAL),
    ],
)
def test_invalid_arguments_rejected_before_launch(fn, args, code):
    rc = getattr(_lib.lib(), fn)(*args)
    assert rc == code
    message = _lib.lib().pt_last_error().decode()
    assert message.startswith(fn)
    with pytest.raises(_lib.HipKernelError, match=fn):
        _lib.check(fn, rc)


def test_empty_inputs_are_no_ops():
    lib = _lib.lib()
    assert lib.pt_swiglu_fwd(None, None, None, 0, 2, None) == _lib.PT_OK
    assert lib.pt_swiglu_bwd(None, None, None, None, None, 5, 2, None) == _lib.PT_OK
    assert lib.pt_adamw_step(None, 0, 0, 1e-3, 0.9, 0.99, 1e-8, 0.0, 1.0, None) == _lib.PT_OK
    assert lib.pt_adamw_step_device_step(None, 0, 0, None, 1e-3, 0.9, 0.99, 1e-8, 0.0, None, 0, None) == _lib.PT_OK
    assert lib.pt_adamw_step_device_step_guarded(None, 0, 0, None, 1e-3, 0.9, 0.99, 1e-8, 0.0, None, 1, None, None, None) == _lib.PT_OK
    assert lib.pt_cross_entropy_shifted_scale_grad(None, 0, 5, 0, 8, 8, None, 5, 1, -100, None, None, 0, 0, None, 2, None) == _lib.PT_OK
    assert lib.pt_last_error() == b""



def test_adamw_tables_skip_empty_tensors_in_one_order():
    import torch

    from picotron_amd import ops

    per = ops.adamw_block_elems()
    params = [torch.zeros(n) for n in (5, 0, per + 1, 0, 3 * per)]
    steps = [torch.zeros(()) for _ in params]
    table, blocks = ops.adamw_table(params, params, params, params)
    step_table = ops.adamw_step_table(params, steps)
    kept = [i for i, p in enumerate(params) if p.numel() > 0]
    assert table.shape == (len(kept), 6) and step_table.shape == (len(kept),)
    assert table[:, 0].tolist() == [params[i].data_ptr() for i in kept]
    assert table[:, 4].tolist() == [params[i].numel() for i in kept]
    assert table[:, 5].tolist() == [0, 1, 3]  # running sums of ceil(numel / block elements)
    assert blocks == 6
    assert step_table.tolist() == [steps[i].data_ptr() for i in kept]


def test_last_error_is_per_thread():
    """pt_last_error is the calling thread's message: a failure in one thread is not cleared
    or overwritten by another thread's calls (the autograd engine issues backward calls from
    its own device thread)."""

    import threading

    lib = _lib.lib()
    first, second = threading.Barrier(2), threading.Barrier(2)
    seen = {}

    def failing():
        seen["a_rc"] = lib.pt_swiglu_fwd(None, None, None, -1, 2, None)
        first.wait()
        second.wait()  # the other thread has failed differently and then succeeded
        seen["a_msg"] = lib.pt_last_error().decode()

    def other():
        first.wait()
        seen["b_fail"] = lib.pt_copy(None, None, 16, None)
        seen["b_fail_msg"] = lib.pt_last_error().decode()
        seen["b_ok"] = lib.pt_swiglu_fwd(None, None, None, 0, 2, None)
        seen["b_msg"] = lib.pt_last_error().decode()
        second.wait()

    threads = [threading.Thread(target=failing), threading.Thread(target=other)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=30)
    assert seen["a_rc"] == _lib.PT_EINVAL and seen["a_msg"].startswith("pt_swiglu_fwd")
    assert seen["b_fail"] == _lib.PT_EINVAL and seen["b_fail_msg"].startswith("pt_copy")
    assert seen["b_ok"] == _lib.PT_OK and seen["b_msg"] == ""
