"""SwiGLU forward/backward parity of the HIP kernels (through the C ABI) with the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import BF16, close, close_fp32, from_npz, randn
from oracle import swiglu as o_swiglu
from picotron_amd import ops

pytestmark = pytest.mark.gpu


def _check(g, u, dy, dtype):
    y = ops.swiglu_fwd(g, u)
    dg, du = ops.swiglu_bwd(dy, g, u)
    y64 = o_swiglu.forward(g, u)
    dg64, du64 = o_swiglu.backward(dy, g, u)
    close(y, y64, dtype)
    close(dg, dg64, dtype)
    close(du, du64, dtype)


def test_quickstart_fp32_matches_reference_fallback(gpu):
    g = randn((128, 256), torch.float32, gpu, 1)
    u = randn((128, 256), torch.float32, gpu, 2)
    dy = randn((128, 256), torch.float32, gpu, 3)
    y = ops.swiglu_fwd(g, u)
    dg, du = ops.swiglu_bwd(dy, g, u)
    fy, fdg, fdu = o_swiglu.fallback_forward_backward(g.cpu(), u.cpu(), dy.cpu())
    close_fp32(y, fy)
    close_fp32(dg, fdg)
    close_fp32(du, fdu)


def test_golden_fixture(gpu):
    f = np.load(GOLDEN / "swiglu_quickstart.npz")
    g, u, dy = (from_npz(f[k], gpu) for k in ("gate", "up", "dy"))
    y = ops.swiglu_fwd(g, u)
    dg, du = ops.swiglu_bwd(dy, g, u)
    for got, key in ((y, "y"), (dg, "dgate"), (du, "dup")):
        close_fp32(got, from_npz(f[key], gpu))


def test_full_config_bf16(gpu):
    # gate, up [16384, 14336] bf16 ~ N(0,1)
    g = randn((16384, 14336), torch.bfloat16, gpu, 11)
    u = randn((16384, 14336), torch.bfloat16, gpu, 12)
    dy = randn((16384, 14336), torch.bfloat16, gpu, 13)
    y = ops.swiglu_fwd(g, u)
    dg, du = ops.swiglu_bwd(dy, g, u)
    # the fp64 oracle evaluated by torch on the GPU, 2048 rows at a time (memory)
    for r in range(0, g.shape[0], 2048):
        sl = slice(r, r + 2048)
        dg64, du64 = o_swiglu.backward(dy[sl], g[sl], u[sl])
        torch.testing.assert_close(y[sl].double(), o_swiglu.forward(g[sl], u[sl]), **BF16)
        torch.testing.assert_close(dg[sl].double(), dg64, **BF16)
        torch.testing.assert_close(du[sl].double(), du64, **BF16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 255, 4097, 1_000_003])
def test_sizes(gpu, dtype, n):
    g = randn((n,), dtype, gpu, n, 3.0)
    u = randn((n,), dtype, gpu, n + 1)
    dy = randn((n,), dtype, gpu, n + 2)
    _check(g, u, dy, dtype)


def test_unaligned_and_special_values(gpu):
    base = randn((4099,), torch.bfloat16, gpu, 5)
    g, u, dy = base[1:4000], base[2:4001], base[3:4002]  # 2-byte offsets: element path
    _check(g, u, dy, torch.bfloat16)
    special = torch.tensor([0.0, -0.0, 1e-30, -100.0, 100.0, -88.0, 88.0, 1.0], device=gpu)
    ones = torch.ones_like(special)
    y = ops.swiglu_fwd(special, ones)
    dg, du = ops.swiglu_bwd(ones, special, ones)
    assert torch.isfinite(y).all() and torch.isfinite(dg).all() and torch.isfinite(du).all()
    close_fp32(y, o_swiglu.forward(special, ones))
    close_fp32(dg, o_swiglu.backward(ones, special, ones)[0])
    assert y[0].item() == 0.0 and dg[0].item() == 0.5


def test_autograd_surface_and_module(gpu):
    import warnings

    from picotron_amd.nn import SwiGLU
    from picotron_amd.nn.triton_kernels import triton_swiglu

    g = randn((3, 40, 700), torch.bfloat16, gpu, 1).requires_grad_(True)
    u = randn((3, 40, 700), torch.bfloat16, gpu, 2).requires_grad_(True)
    dy = randn((3, 40, 700), torch.bfloat16, gpu, 3)
    y = triton_swiglu(g, u)
    y.backward(dy)
    dg64, du64 = o_swiglu.backward(dy, g.detach(), u.detach())
    torch.testing.assert_close(y.double(), o_swiglu.forward(g.detach(), u.detach()), **BF16)
    torch.testing.assert_close(g.grad.double(), dg64, **BF16)
    torch.testing.assert_close(u.grad.double(), du64, **BF16)
    mlp = SwiGLU(64, 160, use_triton_swiglu=True).to(gpu)
    x = randn((2, 5, 64), torch.float32, gpu, 4)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = mlp(x)
    assert not mlp._triton_fallback_warned
    ref = mlp.down_projection(torch.nn.functional.silu(mlp.gate_projection(x)) * mlp.up_projection(x))
    close_fp32(out, ref, rtol=1e-4)
