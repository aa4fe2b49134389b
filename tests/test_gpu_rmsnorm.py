"""RMSNorm forward/backward parity of the HIP kernels (through the C ABI) with the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import BF16, close, close_fp32, from_npz, randn
from oracle import rmsnorm as o_rms
from picotron_amd import ops

pytestmark = pytest.mark.gpu


def _check(x, w, eps, dy, dtype):
    y, rstd = ops.rmsnorm_fwd(x, w, eps)
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    torch.cuda.synchronize()
    y64, r64 = o_rms.forward(x, w, eps)
    dx64, dw64 = o_rms.backward(dy, x, w, eps)
    assert y.dtype == x.dtype and dx.dtype == x.dtype and dw.dtype == w.dtype
    assert rstd.dtype == torch.float32
    close_fp32(rstd, r64)
    close(y, y64, dtype)
    # dx = r*(g*w - x*r^2*dm) cancels when the row is short (cols = 1 cancels exactly up to
    # eps); fp32 error scales with the size of the cancelling terms, not of dx.
    terms = float((dy.double().abs() * w.double().abs()).max() * r64.max()) if dy.numel() else 0.0
    close(dx, dx64, dtype, scale=max(terms, float(dx64.abs().max()) if dx64.numel() else 0.0))
    if w.dtype == torch.float32:
        # an fp32 weight gradient is held to fp32 accuracy: 1e-5 relative, with an absolute
        # floor of 1e-6 of the column's summed magnitudes sum_rows |dy * x * r| (the scale of
        # fp32 accumulation error), so a dropped or doubled partial row cannot pass
        cols = x.size(-1)
        xd, dyd = x.double().reshape(-1, cols), dy.double().reshape(-1, cols)
        mag = (dyd * xd * r64.reshape(-1, 1)).abs().sum(0)
        del xd, dyd
        err = (dw.double() - dw64).abs()
        bound = 1e-5 * dw64.abs() + 1e-6 * mag
        assert bool((err <= bound).all()), f"dW max err/bound {float((err / bound).max())}"
    else:
        close(dw, dw64, w.dtype)
    return y, rstd, dx, dw


def test_quickstart_fp32_matches_reference_fallback(gpu):
    # quickstart config: x [2*64 tokens, 128] fp32, w ~ 1 + 0.02 N(0,1), eps 1e-6
    x = randn((2, 64, 128), torch.float32, gpu, 1)
    w = randn((128,), torch.float32, gpu, 2, 0.02, 1.0)
    dy = randn((2, 64, 128), torch.float32, gpu, 3)
    y, rstd = ops.rmsnorm_fwd(x, w, 1e-6)
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    fy, frstd, fdx, fdw = o_rms.fallback_forward_backward(x.cpu(), w.cpu(), 1e-6, dy.cpu())
    close_fp32(y, fy)
    close_fp32(rstd, frstd)
    close_fp32(dx, fdx)
    close_fp32(dw, fdw)


def test_golden_fixture(gpu):
    f = np.load(GOLDEN / "rmsnorm_quickstart.npz")
    x, w, dy = (from_npz(f[k], gpu) for k in ("x", "w", "dy"))
    y, rstd = ops.rmsnorm_fwd(x, w, float(f["eps"]))
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    for got, key in ((y, "y"), (rstd, "rstd"), (dx, "dx"), (dw, "dw")):
        close_fp32(got, from_npz(f[key], gpu))


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_full_config_bf16(gpu, wdtype):
    # 16384 tokens (8 x 2048) x 4096 bf16, eps 1e-5
    x = randn((8, 2048, 4096), torch.bfloat16, gpu, 11)
    w = randn((4096,), wdtype, gpu, 12, 0.02, 1.0)
    dy = randn((8, 2048, 4096), torch.bfloat16, gpu, 13)
    _check(x, w, 1e-5, dy, torch.bfloat16)


def _ulp(v: torch.Tensor, mantissa_bits: int) -> torch.Tensor:
    """Spacing of the storage grid at each value (bf16: 8 significant bits, fp32: 24)."""

    _, e = torch.frexp(v.double())
    return torch.ldexp(torch.ones_like(v, dtype=torch.float64), e - mantissa_bits)


def test_full_config_mean_square_invariant(gpu):
    # w = 1: mean(y^2) = ms / (ms + eps) per row, to bf16 rounding
    eps = 1e-5
    x = randn((16384, 4096), torch.bfloat16, gpu, 21)
    w = torch.ones(4096, dtype=torch.bfloat16, device=gpu)
    y, rstd = ops.rmsnorm_fwd(x, w, eps)
    ms = x.double().square().mean(-1)
    torch.testing.assert_close(y.double().square().mean(-1), ms / (ms + eps), rtol=5e-3, atol=0)
    torch.testing.assert_close(rstd.double(), 1 / torch.sqrt(ms + eps), rtol=1e-6, atol=0)


@pytest.mark.parametrize("dtype,bits", [(torch.bfloat16, 8), (torch.float32, 24)])
def test_full_config_orthogonality_invariant(gpu, dtype, bits):
    # sum_j dx_j x_j = r * D * dm * eps / (ms + eps) exactly, with dm = mean(dy * w * x):
    # dx is nearly orthogonal to x.  The measured sum may differ only by the rounding of dx
    # to its storage type (per-row sigma from the actual ulps, 8 sigma allowed), by the fp32
    # rstd (2 * 2^-22 relative, times r * D * |dm|) and by the fp32 reduction of dm (which
    # enters as r * D * error(dm); allowed 64 * 2^-24 * r * sum|dy w x|).  The weight is the config's
    # 1 + 0.02 N(0,1): with w = 1, bf16 rounding of dx would correlate with x.
    eps = 1e-5
    x = randn((16384, 4096), dtype, gpu, 21)
    w = randn((4096,), dtype, gpu, 23, 0.02, 1.0)
    dy = randn((16384, 4096), dtype, gpu, 22)
    _, rstd = ops.rmsnorm_fwd(x, w, eps)
    dx, _ = ops.rmsnorm_bwd(dy, x, w, rstd)
    xd, r = x.double(), rstd.double()
    ms = xd.square().mean(-1)
    dm = (dy.double() * w.double() * xd).mean(-1)
    lhs = (dx.double() * xd).sum(-1)
    rhs = r * 4096 * dm * eps / (ms + eps)
    sigma = ((_ulp(dx, bits) ** 2 / 12) * xd.square()).sum(-1).sqrt()
    dot_abs = (dy.double() * w.double() * xd).abs().sum(-1)
    bound = 8 * sigma + 2 * 2.0**-22 * r * 4096 * dm.abs() + 64 * 2.0**-24 * r * dot_abs + 1e-9
    worst = float(((lhs - rhs).abs() / bound).max())
    assert worst <= 1.0, f"orthogonality residual reaches {worst:.2f} of its bound"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "rows,cols",
    [(1, 1), (7, 3), (5, 8), (33, 100), (513, 512), (64, 1000), (3, 4096), (257, 8192),
     (9, 8200), (4, 12288), (3, 16384), (2, 32768), (2, 65536)],
)
def test_shapes(gpu, dtype, rows, cols):
    x = randn((rows, cols), dtype, gpu, rows * 7 + cols)
    w = randn((cols,), dtype, gpu, cols + 1, 0.02, 1.0)
    dy = randn((rows, cols), dtype, gpu, rows + 3 * cols)
    _check(x, w, 1e-5, dy, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mixed_weight_dtypes(gpu, dtype):
    for wdtype in (torch.float32, torch.float16, torch.bfloat16):
        x = randn((37, 640), dtype, gpu, 5)
        w = randn((640,), wdtype, gpu, 6, 0.02, 1.0)
        dy = randn((37, 640), dtype, gpu, 7)
        _check(x, w, 1e-6, dy, dtype)


def test_strided_and_unaligned_rows(gpu):
    dtype = torch.bfloat16
    big = randn((300, 4096 + 24), dtype, gpu, 8)
    x = big[:, 8 : 8 + 4096]  # row stride 4120, base offset 16 bytes: aligned vectors
    w = randn((4096,), dtype, gpu, 9, 0.02, 1.0)
    dy = randn((300, 4096), dtype, gpu, 10)
    _check(x, w, 1e-5, dy, dtype)
    xu = big[:, 1 : 1 + 4096]  # offset by one element: element-wise path
    _check(xu, w, 1e-5, dy, dtype)
    xo = randn((300, 4095), dtype, gpu, 11)  # odd hidden size
    _check(xo, randn((4095,), dtype, gpu, 12, 0.02, 1.0), 1e-5, randn((300, 4095), dtype, gpu, 13), dtype)


def test_empty_and_partial_gradients(gpu):
    x = torch.empty((0, 256), dtype=torch.bfloat16, device=gpu)
    w = randn((256,), torch.bfloat16, gpu, 1, 0.02, 1.0)
    y, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    dx, dw = ops.rmsnorm_bwd(x, x, w, rstd)
    assert y.shape == (0, 256) and dx.shape == (0, 256)
    assert torch.equal(dw, torch.zeros_like(dw))
    x = randn((10, 256), torch.bfloat16, gpu, 2)
    dy = randn((10, 256), torch.bfloat16, gpu, 3)
    y, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    dx_only, none_w = ops.rmsnorm_bwd(dy, x, w, rstd, need_dw=False)
    none_x, dw_only = ops.rmsnorm_bwd(dy, x, w, rstd, need_dx=False)
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    assert none_w is None and none_x is None
    assert torch.equal(dx_only, dx) and torch.equal(dw_only, dw)


def test_weight_gradient_is_deterministic(gpu):
    x = randn((16384, 4096), torch.bfloat16, gpu, 31)
    w = randn((4096,), torch.float32, gpu, 32, 0.02, 1.0)
    dy = randn((16384, 4096), torch.bfloat16, gpu, 33)
    _, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    runs = [ops.rmsnorm_bwd(dy, x, w, rstd) for _ in range(3)]
    for dx, dw in runs[1:]:
        assert torch.equal(dx, runs[0][0]) and torch.equal(dw, runs[0][1])


def test_autograd_surface_and_module(gpu):
    import warnings

    from picotron_amd.nn import RMSNorm
    from picotron_amd.nn.triton_kernels import triton_rms_norm

    x = randn((4, 50, 1024), torch.bfloat16, gpu, 41).requires_grad_(True)
    w = randn((1024,), torch.float32, gpu, 42, 0.02, 1.0).requires_grad_(True)
    dy = randn((4, 50, 1024), torch.bfloat16, gpu, 43)
    y = triton_rms_norm(x, w, 1e-6)
    y.backward(dy)
    y64, _ = o_rms.forward(x.detach(), w.detach(), 1e-6)
    dx64, dw64 = o_rms.backward(dy, x.detach(), w.detach(), 1e-6)
    torch.testing.assert_close(y.double(), y64, **BF16)
    torch.testing.assert_close(x.grad.double(), dx64, **BF16)
    close_fp32(w.grad, dw64, rtol=1e-4)
    norm = RMSNorm(1024, use_triton_rmsnorm=True).to(gpu)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = norm(x.detach().float())
    assert not norm._triton_fallback_warned
    ref, _ = o_rms.forward(x.detach().float(), norm.weight.detach(), norm.eps)
    close_fp32(out, ref)


def test_banner_rows_report_the_hip_kernels(gpu):
    from picotron_amd.config import TritonKernelsConfig
    from picotron_amd.hardware import kernel_status_rows

    rows = kernel_status_rows(TritonKernelsConfig(rmsnorm=True, swiglu=True), device=gpu)
    assert rows[0] == ("Triton kernels", "active: rmsnorm, swiglu")
    assert rows[1] == ("Triton status", "rmsnorm=real swiglu=real rope=real "
                       "attention=fallback cross_entropy=real adamw=real")
