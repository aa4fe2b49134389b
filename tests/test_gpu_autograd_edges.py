"""Autograd edge cases of the fused ops: the upstream gradient of ``out.sum()`` is a
stride-0 expanded tensor, and ``out[..., ::2].sum()`` a strided one; the fused backward must
give the fallback's gradients (fp32, tolerance of the fp32 parity tests)."""

from __future__ import annotations

import pytest
import torch

from gpu_util import close_fp32, randn
from oracle import rope as o_rope
from picotron_amd.nn.triton_kernels import (
    rms_norm_with_pytorch_forward,
    triton_apply_rotary_embedding,
    triton_residual_rms_norm,
    triton_rms_norm,
    swiglu_with_pytorch_forward,
    triton_swiglu,
)
from picotron_amd.nn.rope import apply_rotary_embedding

pytestmark = pytest.mark.gpu

REDUCTIONS = {
    "sum": lambda y: y.sum(),  # expanded (stride 0) upstream gradient
    "strided": lambda y: (y[..., ::2] * 1.5).sum(),  # gradient with zeros at odd columns
}


def _grads(fn, *inputs):
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    out = fn(*leaves)
    return out, leaves


@pytest.mark.parametrize("reduce", list(REDUCTIONS))
def test_rmsnorm(gpu, reduce):
    x = randn((6, 33, 200), torch.float32, gpu, 1)
    w = randn((200,), torch.float32, gpu, 2, 0.1, 1.0)
    y_f, (xf, wf) = _grads(lambda a, b: triton_rms_norm(a, b, 1e-6), x, w)
    y_r, (xr, wr) = _grads(lambda a, b: rms_norm_with_pytorch_forward(a, b, 1e-6), x, w)
    REDUCTIONS[reduce](y_f).backward()
    REDUCTIONS[reduce](y_r).backward()
    close_fp32(xf.grad, xr.grad, scale=float(xr.grad.abs().max()) * 10)
    close_fp32(wf.grad, wr.grad)


@pytest.mark.parametrize("reduce", list(REDUCTIONS))
def test_residual_rmsnorm(gpu, reduce):
    x, r = randn((5, 64), torch.float32, gpu, 3), randn((5, 64), torch.float32, gpu, 4)
    w = randn((64,), torch.float32, gpu, 5, 0.1, 1.0)
    outs, (xf, rf, wf) = _grads(lambda a, b, c: triton_residual_rms_norm(a, b, c, 1e-6), x, r, w)

    def ref(a, b, c):
        h = a + b
        return h, rms_norm_with_pytorch_forward(h, c, 1e-6)

    refs, (xr, rr, wr) = _grads(ref, x, r, w)
    (REDUCTIONS[reduce](outs[0]) + REDUCTIONS[reduce](outs[1])).backward()
    (REDUCTIONS[reduce](refs[0]) + REDUCTIONS[reduce](refs[1])).backward()
    for a, b in ((xf, xr), (rf, rr), (wf, wr)):
        close_fp32(a.grad, b.grad, scale=float(b.grad.abs().max()) * 10)


@pytest.mark.parametrize("reduce", list(REDUCTIONS))
def test_swiglu(gpu, reduce):
    g, u = randn((7, 130), torch.float32, gpu, 6), randn((7, 130), torch.float32, gpu, 7)
    y_f, (gf, uf) = _grads(triton_swiglu, g, u)
    y_r, (gr, ur) = _grads(swiglu_with_pytorch_forward, g, u)
    REDUCTIONS[reduce](y_f).backward()
    REDUCTIONS[reduce](y_r).backward()
    close_fp32(gf.grad, gr.grad)
    close_fp32(uf.grad, ur.grad)


@pytest.mark.parametrize("reduce", list(REDUCTIONS))
def test_rope(gpu, reduce):
    x = randn((2, 3, 19, 32), torch.float32, gpu, 8)
    cos, sin = o_rope.tables(19, 32, 10_000.0, device=gpu)
    y_f, (xf,) = _grads(lambda a: triton_apply_rotary_embedding(a, cos, sin), x)
    y_r, (xr,) = _grads(lambda a: apply_rotary_embedding(a, cos, sin), x)
    REDUCTIONS[reduce](y_f).backward()
    REDUCTIONS[reduce](y_r).backward()
    close_fp32(xf.grad, xr.grad)


def test_repeated_backward_with_retain_graph(gpu):
    """RMSNorm (plain and with the residual add), SwiGLU and RoPE keep their saved tensors
    intact through a backward: a second backward through the retained graph (as torch's own
    ops allow) gives bit-identical gradients."""

    x = randn((4, 40, 128), torch.float32, gpu, 20)
    r = randn((4, 40, 128), torch.float32, gpu, 21)
    w = randn((128,), torch.float32, gpu, 22, 0.1, 1.0)
    g, u = randn((4, 40, 256), torch.float32, gpu, 23), randn((4, 40, 256), torch.float32, gpu, 24)
    q = randn((2, 4, 40, 32), torch.float32, gpu, 25)
    cos, sin = o_rope.tables(40, 32, 10_000.0, device=gpu)
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, r, w, g, u, q)]
    xl, rl, wl, gl, ul, ql = leaves
    h, y = triton_residual_rms_norm(xl, rl, wl, 1e-6)
    out = (triton_rms_norm(y, wl, 1e-6) * 0.5 + h).sum() + (triton_swiglu(gl, ul) ** 2).sum()
    out = out + (triton_apply_rotary_embedding(ql, cos, sin) * 1.25).sum()
    first = torch.autograd.grad(out, leaves, retain_graph=True)
    second = torch.autograd.grad(out, leaves)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def _first_and_second(fn, inputs, v, weights):
    """First-order gradients of (fn(*inputs) * v).sum() with create_graph=True, then the
    gradient of sum(g_i * weights_i) with respect to the inputs and v."""

    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    vl = v.detach().clone().requires_grad_(True)
    out = fn(*leaves)
    outs = out if isinstance(out, tuple) else (out,)
    total = sum((o * vl).sum() for o in outs)
    first = torch.autograd.grad(total, leaves, create_graph=True)
    z = sum((g * a).sum() for g, a in zip(first, weights))
    second = torch.autograd.grad(z, leaves + [vl], allow_unused=True)
    return [g.detach() for g in first], second


def _close_all(a_list, b_list):
    for a, b in zip(a_list, b_list):
        if a is None or b is None:
            assert a is None and b is None or float((a if a is not None else b).abs().max()) == 0.0
            continue
        close_fp32(a, b, scale=float(b.abs().max()) * 10 + 1e-30)


@pytest.mark.parametrize("op", ["rmsnorm", "residual_rmsnorm", "swiglu", "rope"])
def test_higher_order_gradients_follow_the_reference_formulas(gpu, op):
    """With create_graph=True the fused ops' backwards build a graph as the reference's eager
    backwards do (rmsnorm.py:110-134, swiglu.py:71-81; RoPE's backward is a rotation), so
    second-order gradients equal the reference path's instead of treating the kernel's
    gradient as a constant."""

    if op == "rmsnorm":
        x, w = randn((3, 17, 96), torch.float32, gpu, 30), randn((96,), torch.float32, gpu, 31, 0.1, 1.0)
        inputs, v = [x, w], randn((3, 17, 96), torch.float32, gpu, 32)
        fused = lambda a, b: triton_rms_norm(a, b, 1e-6)  # noqa: E731
        ref = lambda a, b: rms_norm_with_pytorch_forward(a, b, 1e-6)  # noqa: E731
    elif op == "residual_rmsnorm":
        x, r = randn((3, 17, 96), torch.float32, gpu, 33), randn((3, 17, 96), torch.float32, gpu, 34)
        w = randn((96,), torch.float32, gpu, 35, 0.1, 1.0)
        inputs, v = [x, r, w], randn((3, 17, 96), torch.float32, gpu, 36)
        fused = lambda a, b, c: triton_residual_rms_norm(a, b, c, 1e-6)  # noqa: E731

        def ref(a, b, c):
            h = a + b
            return h, rms_norm_with_pytorch_forward(h, c, 1e-6)
    elif op == "swiglu":
        inputs = [randn((5, 70), torch.float32, gpu, 37), randn((5, 70), torch.float32, gpu, 38)]
        v = randn((5, 70), torch.float32, gpu, 39)
        fused, ref = triton_swiglu, swiglu_with_pytorch_forward
    else:
        inputs, v = [randn((2, 3, 19, 32), torch.float32, gpu, 40)], randn((2, 3, 19, 32), torch.float32, gpu, 41)
        cos, sin = o_rope.tables(19, 32, 10_000.0, device=gpu)
        fused = lambda a: triton_apply_rotary_embedding(a, cos, sin)  # noqa: E731
        ref = lambda a: apply_rotary_embedding(a, cos, sin)  # noqa: E731
    weights = [randn(t.shape, torch.float32, gpu, 50 + i) for i, t in enumerate(inputs)]
    first_f, second_f = _first_and_second(fused, inputs, v, weights)
    first_r, second_r = _first_and_second(ref, inputs, v, weights)
    _close_all(first_f, first_r)
    _close_all(second_f, second_r)
    # the second-order gradient reaches the upstream gradient v in every op
    assert second_f[-1] is not None and float(second_f[-1].abs().max()) > 0
