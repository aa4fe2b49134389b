"""pt_rmsnorm_bwd_noalloc (the RMSNorm backward whose weight-gradient partials live in the
library's static device scratch instead of a caller workspace) against pt_rmsnorm_bwd,
through the C ABI: two calls in a row, the second on a smaller input, so that partial rows
left in the scratch by the first call would show in the second's weight gradient."""

from __future__ import annotations

import pytest
import torch

from gpu_util import randn
from picotron_amd import _lib, ops

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _noalloc(dy, x, w, rstd, need_dx=True, need_dw=True):
    rows, cols = x.shape
    dx = torch.empty_like(x) if need_dx else None
    dw = torch.empty(cols, dtype=w.dtype, device=x.device) if need_dw else None
    _lib.call(
        "pt_rmsnorm_bwd_noalloc",
        dy.data_ptr(), cols, x.data_ptr(), cols, w.data_ptr(), rstd.data_ptr(),
        None if dx is None else dx.data_ptr(), cols, None if dw is None else dw.data_ptr(),
        rows, cols, ops.dtype_code(x.dtype), ops.dtype_code(w.dtype),
        torch.cuda.current_stream(x.device).cuda_stream,
    )
    return dx, dw


def _inputs(rows, cols, dtype, wdtype, device, seed):
    x = randn((rows, cols), dtype, device, seed)
    dy = randn((rows, cols), dtype, device, seed + 1)
    w = randn((cols,), wdtype, device, seed + 2, 0.02, 1.0)
    _, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    return x, dy, w, rstd


@pytest.mark.parametrize(
    "first,second",
    [
        # the headline shape (8 MiB of partials), then a smaller one with fewer partial rows
        ((16384, 4096, torch.bfloat16, torch.bfloat16), (1000, 1024, torch.bfloat16, torch.bfloat16)),
        # fp32 weight gradient, then a ragged row length on the element-wise path
        ((4096, 2048, torch.bfloat16, torch.float32), (37, 1001, torch.float32, torch.float32)),
    ],
)
def test_matches_the_workspace_entry_point_on_consecutive_calls(gpu, first, second):
    for seed, (rows, cols, dtype, wdtype) in zip((11, 21), (first, second)):
        print(f"noalloc case rows={rows} cols={cols} x={dtype} w={wdtype}", flush=True)
        x, dy, w, rstd = _inputs(rows, cols, dtype, wdtype, gpu, seed)
        dx_ref, dw_ref = ops.rmsnorm_bwd(dy, x, w, rstd)
        dx, dw = _noalloc(dy, x, w, rstd)
        torch.cuda.synchronize()
        # same kernels, same grid, same summation order: bitwise equal
        assert torch.equal(dx, dx_ref)
        assert torch.equal(dw, dw_ref)
        # and both are right (the fp64 formula of the reference backward)
        xd, dyd = x.double(), dy.double()
        r = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-5)
        dw64 = (dyd * xd * r).sum(0)
        tol = 1e-5 if wdtype == torch.float32 else 1.6e-2
        scale = float((dyd * xd * r).abs().sum(0).max())
        torch.testing.assert_close(dw.double(), dw64, rtol=tol, atol=1e-6 * scale if wdtype == torch.float32 else 2e-2)


def test_input_gradient_only_and_empty_batch(gpu):
    x, dy, w, rstd = _inputs(512, 4096, torch.bfloat16, torch.bfloat16, gpu, 31)
    dx, dw = _noalloc(dy, x, w, rstd, need_dw=False)
    dx_ref, _ = ops.rmsnorm_bwd(dy, x, w, rstd, need_dw=False)
    assert dw is None and torch.equal(dx, dx_ref)
    # no rows: the weight gradient is a sum over nothing
    e = torch.empty(0, 256, dtype=torch.bfloat16, device=gpu)
    w = torch.ones(256, dtype=torch.bfloat16, device=gpu)
    _, dw = _noalloc(e, e, w, torch.empty(0, dtype=torch.float32, device=gpu), need_dx=False)
    torch.cuda.synchronize()
    assert torch.count_nonzero(dw) == 0


def test_partials_beyond_the_scratch_are_rejected_before_launch(gpu):
    rows, cols = 16384, 16384  # 512 partial rows of 16384 fp32 = 32 MiB
    need = _lib.lib().pt_rmsnorm_bwd_workspace_bytes(rows, cols, _lib.PT_BFLOAT16)
    assert need > SCRATCH_BYTES
    # full-size buffers, so that nothing could be read out of bounds even if a launch happened
    dy, x, dx = (torch.zeros(rows, cols, dtype=torch.bfloat16, device=gpu) for _ in range(3))
    w = torch.ones(cols, dtype=torch.bfloat16, device=gpu)
    dw = torch.empty(cols, dtype=torch.bfloat16, device=gpu)
    rstd = torch.ones(rows, dtype=torch.float32, device=gpu)
    rc = _lib.lib().pt_rmsnorm_bwd_noalloc(
        dy.data_ptr(), cols, x.data_ptr(), cols, w.data_ptr(), rstd.data_ptr(), dx.data_ptr(), cols,
        dw.data_ptr(), rows, cols, _lib.PT_BFLOAT16, _lib.PT_BFLOAT16,
        torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == _lib.PT_EUNSUPPORTED
    message = _lib.lib().pt_last_error().decode()
    assert "static scratch" in message and str(need) in message


def test_replays_of_a_captured_call_match_the_workspace_entry_point(gpu):
    # The first call on a device looks up the scratch's address (and is refused inside a
    # capture), so one eager call comes first; the captured call then replays on new inputs
    # written by eager work between the replays.
    rows, cols = 4096, 4096
    x, dy, w, rstd = _inputs(rows, cols, torch.bfloat16, torch.bfloat16, gpu, 41)
    dx = torch.empty_like(x)
    dw = torch.empty(cols, dtype=w.dtype, device=gpu)
    stream = torch.cuda.Stream()

    def call():
        _lib.call(
            "pt_rmsnorm_bwd_noalloc",
            dy.data_ptr(), cols, x.data_ptr(), cols, w.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
            cols, dw.data_ptr(), rows, cols, _lib.PT_BFLOAT16, _lib.PT_BFLOAT16,
            torch.cuda.current_stream(gpu).cuda_stream,
        )

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call()
    for replay in range(3):
        xn, dyn, _, _ = _inputs(rows, cols, torch.bfloat16, torch.bfloat16, gpu, 50 + replay)
        x.copy_(xn)
        dy.copy_(dyn)
        _, r = ops.rmsnorm_fwd(x, w, 1e-5)
        rstd.copy_(r)
        dx_ref, dw_ref = ops.rmsnorm_bwd(dy, x, w, rstd)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_ref), f"replay {replay}: dx"
        assert torch.equal(dw, dw_ref), f"replay {replay}: dW"
