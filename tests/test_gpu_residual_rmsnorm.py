"""Residual add + RMSNorm fusion (decoder block: h = x + attention(...), then mlp_norm(h)):
parity of the fused HIP kernels (through the C ABI) with the oracle and torch."""

from __future__ import annotations

import pytest
import torch

from gpu_util import close, close_fp32, randn
from oracle import rmsnorm as o_rms
from picotron_amd import ops

pytestmark = pytest.mark.gpu


def _case(gpu, shape, dtype, wdtype, seed):
    x = randn(shape, dtype, gpu, seed)
    r = randn(shape, dtype, gpu, seed + 1)
    w = randn((shape[-1],), wdtype, gpu, seed + 2, 0.02, 1.0)
    dy = randn(shape, dtype, gpu, seed + 3)
    dh_in = randn(shape, dtype, gpu, seed + 4)
    return x, r, w, dy, dh_in


def _check(x, r, w, dy, dh_in, eps, dtype):
    h, y, rstd = ops.residual_rmsnorm_fwd(x, r, w, eps)
    assert torch.equal(h, x + r)  # the stored sum is torch's add, bit for bit
    oh, y64, r64 = o_rms.residual_forward(x, r, w, eps)
    close_fp32(rstd, r64)
    close(y, y64, dtype)
    dh, dw = ops.residual_rmsnorm_bwd(dy, dh_in, h, w, rstd)
    dh64, dw64 = o_rms.residual_backward(dy, dh_in, oh, w, eps)
    terms = float((dy.double().abs() * w.double().abs()).max() * r64.max()) + float(dh_in.double().abs().max())
    close(dh, dh64, dtype, scale=max(terms, float(dh64.abs().max())))
    close(dw, dw64, w.dtype if w.dtype != torch.float32 else dtype)
    return h, y, rstd, dh, dw


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 8), (7, 64), (33, 4096), (5, 1000), (300, 2048), (4, 8192)])
def test_shapes(gpu, dtype, rows, cols):
    _check(*_case(gpu, (rows, cols), dtype, dtype, rows + cols), 1e-5, dtype)


def test_full_config_bf16(gpu):
    # decoder-block shape [8 x 2048 tokens, 4096] bf16 with the module's fp32 weight
    x, r, w, dy, dh_in = _case(gpu, (8, 2048, 4096), torch.bfloat16, torch.float32, 40)
    _check(x, r, w, dy, dh_in, 1e-5, torch.bfloat16)


def test_matches_unfused_kernels(gpu):
    # fused forward == add then pt_rmsnorm_fwd; fused backward == pt_rmsnorm_bwd + dh_in
    x, r, w, dy, dh_in = _case(gpu, (512, 4096), torch.float32, torch.float32, 50)
    h, y, rstd = ops.residual_rmsnorm_fwd(x, r, w, 1e-5)
    y2, rstd2 = ops.rmsnorm_fwd(x + r, w, 1e-5)
    assert torch.equal(y, y2) and torch.equal(rstd, rstd2)
    dh, dw = ops.residual_rmsnorm_bwd(dy, dh_in, h, w, rstd)
    dx2, dw2 = ops.rmsnorm_bwd(dy, h, w, rstd)
    assert torch.equal(dw, dw2)
    close_fp32(dh, dx2 + dh_in)


def test_in_place_accumulation_and_no_incoming_gradient(gpu):
    x, r, w, dy, dh_in = _case(gpu, (64, 1024), torch.bfloat16, torch.bfloat16, 60)
    h, y, rstd = ops.residual_rmsnorm_fwd(x, r, w, 1e-6)
    expected, dw_e = ops.residual_rmsnorm_bwd(dy, dh_in, h, w, rstd)
    acc = dh_in.clone()
    out, dw = ops.residual_rmsnorm_bwd(dy, acc, h, w, rstd, out=acc)  # dh written over dh_in
    assert out.data_ptr() == acc.data_ptr()
    assert torch.equal(acc, expected) and torch.equal(dw, dw_e)
    plain, _ = ops.residual_rmsnorm_bwd(dy, None, h, w, rstd)
    dx, _ = ops.rmsnorm_bwd(dy, h, w, rstd)
    assert torch.equal(plain, dx)


def test_rejects_aliasing_outputs(gpu):
    from picotron_amd import _lib

    x = torch.randn(4, 64, device=gpu)
    w = torch.ones(64, device=gpu)
    rstd = torch.empty(4, device=gpu)
    y = torch.empty_like(x)
    lib = _lib.lib()
    p = lambda t: t.data_ptr()  # noqa: E731
    rc = lib.pt_residual_rmsnorm_fwd(p(x), 64, p(x), 64, p(w), p(x), 64, p(y), 64, p(rstd), 4, 64,
                                     1e-6, 0, 0, None)
    assert rc == _lib.PT_EINVAL and b"alias" in lib.pt_last_error()


def test_autograd_decoder_block(gpu):
    # out = h + mlp(norm(h)) with h = x + attn: autograd through the fused Function against
    # fp64 autograd of the unfused graph
    from picotron_amd.nn import RMSNorm

    shape = (2, 33, 256)
    x0, r0, _, _, _ = _case(gpu, shape, torch.bfloat16, torch.float32, 70)
    norm = RMSNorm(256, eps=1e-6, use_triton_rmsnorm=True).to(gpu)
    with torch.no_grad():
        norm.weight.copy_(randn((256,), torch.float32, gpu, 72, 0.02, 1.0))
    proj = randn((256, 256), torch.float32, gpu, 73, 0.05)
    x = x0.clone().requires_grad_(True)
    r = r0.clone().requires_grad_(True)
    h, y = norm.add_and_norm(x, r)
    assert not norm._triton_fallback_warned
    out = h + (y.float() @ proj).to(h.dtype)
    g = randn(shape, torch.bfloat16, gpu, 74)
    out.backward(g)
    xd, rd = x0.double().requires_grad_(True), r0.double().requires_grad_(True)
    wd = norm.weight.detach().double().requires_grad_(True)
    hd = (x0.float() + r0.float()).to(torch.bfloat16).double() + (xd + rd - (xd + rd).detach())
    yd = hd * torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-6) * wd
    outd = hd + yd @ proj.double()
    outd.backward(g.double())
    close(x.grad, xd.grad, torch.bfloat16)
    close(r.grad, rd.grad, torch.bfloat16)
    close(norm.weight.grad, wd.grad, torch.bfloat16)  # dy reaches the norm rounded to bf16
