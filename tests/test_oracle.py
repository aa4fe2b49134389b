"""Pins for the oracle: each function checked against something other than its own formula
(reference known-answer tests, torch library routines, gradcheck, closed forms, invariants).
CPU only."""

from __future__ import annotations

import math

import pytest
import torch
from torch.nn import functional as F

from oracle import adamw as o_adamw
from oracle import cross_entropy as o_ce
from oracle import rmsnorm as o_rms
from oracle import rope as o_rope
from oracle import swiglu as o_swiglu

# ------------------------------------------------------------------ RMSNorm


def _native_rms_norm(x, w, eps):
    # the formula of the reference test (tests/test_triton_rmsnorm_backward.py:8-10)
    return x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + eps) * w


def test_rmsnorm_oracle_matches_autograd_of_native_formula_reference_case():
    # reference tests/test_triton_rmsnorm_backward.py:13-32: seed 23, [2,3,8], eps 1e-6
    torch.manual_seed(23)
    eps = 1e-6
    dy = torch.randn(2, 3, 8, dtype=torch.float32)
    x = torch.randn(2, 3, 8, dtype=torch.float32, requires_grad=True)
    w = torch.randn(8, dtype=torch.float32, requires_grad=True)
    y_native = _native_rms_norm(x, w, eps)
    (y_native * dy).sum().backward()
    y, _ = o_rms.forward(x.detach(), w.detach(), eps, torch.float32)
    dx, dw = o_rms.backward(dy, x.detach(), w.detach(), eps, torch.float32)
    torch.testing.assert_close(y, y_native.detach(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(dx, x.grad, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(dw, w.grad, rtol=1e-5, atol=1e-6)


def test_rmsnorm_oracle_backward_gradcheck_fp64():
    torch.manual_seed(0)
    eps = 1e-3
    x = torch.randn(3, 5, dtype=torch.float64, requires_grad=True)
    w = torch.randn(5, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(3, 5, dtype=torch.float64)

    def f(x, w):
        return (o_rms.forward(x, w, eps)[0] * dy).sum()

    assert torch.autograd.gradcheck(f, (x, w))
    gx, gw = torch.autograd.grad(f(x, w), (x, w))
    dx, dw = o_rms.backward(dy, x.detach(), w.detach(), eps)
    torch.testing.assert_close(dx, gx, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dw, gw, rtol=1e-10, atol=1e-12)


def test_rmsnorm_oracle_invariants():
    torch.manual_seed(1)
    eps = 1e-5
    x = torch.randn(64, 32, dtype=torch.float64)
    ones = torch.ones(32, dtype=torch.float64)
    y, rstd = o_rms.forward(x, ones, eps)
    ms = x.square().mean(-1)
    # w = 1: mean(y^2) = ms / (ms + eps)
    torch.testing.assert_close(y.square().mean(-1), ms / (ms + eps), rtol=1e-12, atol=0)
    torch.testing.assert_close(rstd, 1 / torch.sqrt(ms + eps), rtol=1e-14, atol=0)
    # scale invariance as eps -> 0
    y2, _ = o_rms.forward(7.0 * x, ones, 0.0)
    y1, _ = o_rms.forward(x, ones, 0.0)
    torch.testing.assert_close(y2, y1, rtol=1e-12, atol=1e-12)
    # sum_j dx_j x_j = r * D * dm * eps / (ms + eps)
    w = 1 + 0.02 * torch.randn(32, dtype=torch.float64)
    dy = torch.randn(64, 32, dtype=torch.float64)
    dx, dw = o_rms.backward(dy, x, w, eps)
    r = 1 / torch.sqrt(ms + eps)
    dm = (dy * w * x).mean(-1)
    torch.testing.assert_close((dx * x).sum(-1), r * 32 * dm * eps / (ms + eps), rtol=1e-8, atol=1e-12)
    # dW = sum_rows(dy * y / w)
    y, _ = o_rms.forward(x, w, eps)
    torch.testing.assert_close(dw, (dy * y / w).sum(0), rtol=1e-10, atol=1e-10)


def test_rmsnorm_fallback_restatement_matches_oracle():
    torch.manual_seed(2)
    x = torch.randn(16, 24)
    w = 1 + 0.02 * torch.randn(24)
    dy = torch.randn(16, 24)
    y, rstd, dx, dw = o_rms.fallback_forward_backward(x, w, 1e-6, dy)
    y64, r64 = o_rms.forward(x, w, 1e-6)
    dx64, dw64 = o_rms.backward(dy, x, w, 1e-6)
    torch.testing.assert_close(y.double(), y64, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(rstd.double(), r64, rtol=1e-6, atol=0)
    torch.testing.assert_close(dx.double(), dx64, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(dw.double(), dw64, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ SwiGLU


def test_swiglu_oracle_matches_torch_silu_and_autograd_reference_case():
    # reference tests/test_triton_swiglu_backward.py:9-26: seed 31, [2,3,7] fp64, 1e-10
    torch.manual_seed(31)
    dy = torch.randn(2, 3, 7, dtype=torch.float64)
    g = torch.randn(2, 3, 7, dtype=torch.float64, requires_grad=True)
    u = torch.randn(2, 3, 7, dtype=torch.float64, requires_grad=True)
    native = F.silu(g) * u
    (native * dy).sum().backward()
    torch.testing.assert_close(o_swiglu.forward(g.detach(), u.detach()), native.detach(), rtol=1e-10, atol=1e-10)
    dg, du = o_swiglu.backward(dy, g.detach(), u.detach())
    torch.testing.assert_close(dg, g.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(du, u.grad, rtol=1e-10, atol=1e-10)


def test_swiglu_oracle_gradcheck_and_special_values():
    torch.manual_seed(3)
    g = torch.randn(4, 6, dtype=torch.float64, requires_grad=True)
    u = torch.randn(4, 6, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: o_swiglu.forward(a, b), (g, u))
    zero = torch.zeros(3, dtype=torch.float64)
    one = torch.ones(3, dtype=torch.float64)
    assert torch.equal(o_swiglu.forward(zero, one), zero)  # silu(0) = 0
    dg, du = o_swiglu.backward(one, zero, one)
    torch.testing.assert_close(dg, 0.5 * one)  # silu'(0) = 1/2
    assert torch.equal(du, zero)
    big = torch.tensor([40.0], dtype=torch.float64)
    torch.testing.assert_close(o_swiglu.forward(big, torch.ones(1, dtype=torch.float64)), big)


def test_swiglu_fallback_restatement_matches_oracle():
    torch.manual_seed(4)
    g, u, dy = torch.randn(3, 50, 20).unbind(0)
    y, dg, du = o_swiglu.fallback_forward_backward(g, u, dy)
    torch.testing.assert_close(y.double(), o_swiglu.forward(g, u), rtol=1e-5, atol=1e-6)
    dg64, du64 = o_swiglu.backward(dy, g, u)
    torch.testing.assert_close(dg.double(), dg64, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(du.double(), du64, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ RoPE


def test_rope_tables_known_values():
    cos, sin = o_rope.tables(4, 128, 500_000.0)
    inv = torch.atan2(sin[1], cos[1])  # angle at position 1 = inv_freq
    assert abs(inv[0].item() - 1.0) < 1e-7
    assert abs(inv[1].item() - 0.8146172339) < 1e-6  # 5e5 ** (-2/128)
    assert abs(inv[1].item() - 500_000.0 ** (-2 / 128)) < 1e-6
    assert torch.equal(cos[0], torch.ones(64)) and torch.equal(sin[0], torch.zeros(64))


@pytest.mark.parametrize("layout", ["interleaved", "rotate_half"])
def test_rope_rotation_closed_form_and_invariants(layout):
    torch.manual_seed(5)
    d = 8
    cos, sin = o_rope.tables(6, d, 10_000.0)
    # basis vector of pair 1 at position 3 rotates to (cos a, sin a)
    e = torch.zeros(1, 1, 6, d, dtype=torch.float64)
    i0, i1 = (2, 3) if layout == "interleaved" else (1, 1 + d // 2)
    e[..., 3, i0] = 1.0
    out = o_rope.rotate(e, cos, sin, layout)
    torch.testing.assert_close(out[0, 0, 3, i0], cos[3, 1].double())
    torch.testing.assert_close(out[0, 0, 3, i1], sin[3, 1].double())
    x = torch.randn(2, 3, 6, d, dtype=torch.float64)
    y = o_rope.rotate(x, cos, sin, layout)
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1))  # norm preserved
    torch.testing.assert_close(y[..., 0, :], x[..., 0, :])  # position 0 is identity
    back = o_rope.rotate(y, cos, sin, layout, inverse=True)
    torch.testing.assert_close(back, x)  # inverse o forward = identity
    # the inverse is the backward: <rotate(x), dy> = <x, inverse(dy)>
    dy = torch.randn_like(x)
    torch.testing.assert_close((y * dy).sum(), (x * o_rope.rotate(dy, cos, sin, layout, inverse=True)).sum())


def test_rope_relative_position_reference_case():
    # reference tests/test_rope.py:10-23
    torch.manual_seed(0)
    d = 8
    q = torch.randn(1, 1, 1, d).expand(-1, -1, 12, -1).clone()
    k = torch.randn(1, 1, 1, d).expand(-1, -1, 12, -1).clone()
    cos, sin = o_rope.tables(12, d, 10_000.0)
    rq = o_rope.rotate(q, cos, sin, compute=torch.float32)
    rk = o_rope.rotate(k, cos, sin, compute=torch.float32)
    torch.testing.assert_close((rq[:, :, 2] * rk[:, :, 5]).sum(), (rq[:, :, 6] * rk[:, :, 9]).sum())


def test_rope_layouts_related_by_permutation():
    torch.manual_seed(6)
    d = 16
    cos, sin = o_rope.tables(5, d, 10_000.0)
    x = torch.randn(2, 3, 5, d, dtype=torch.float64)
    perm = torch.cat((torch.arange(0, d, 2), torch.arange(1, d, 2)))  # evens then odds
    torch.testing.assert_close(
        o_rope.rotate(x[..., perm], cos, sin, "rotate_half"),
        o_rope.rotate(x, cos, sin, "interleaved")[..., perm],
    )


def test_rope_fallback_restatement_matches_oracle():
    torch.manual_seed(7)
    cos, sin = o_rope.tables(5, 8, 10_000.0)
    x = torch.randn(2, 3, 5, 8)
    dy = torch.randn(2, 3, 5, 8)
    y, dx = o_rope.fallback_forward_backward(x, cos, sin, dy)
    torch.testing.assert_close(y.double(), o_rope.rotate(x, cos, sin), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(dx.double(), o_rope.rotate(dy, cos, sin, inverse=True), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ cross-entropy


def test_cross_entropy_known_answer_reference_case():
    # reference tests/test_triton_ce_adamw.py:15-24; mean 1.2887259920 (closed form)
    logits = torch.tensor([[2.0, 0.0, -1.0], [0.5, 1.5, -0.5]], dtype=torch.float64)
    targets = torch.tensor([0, 2])
    loss, _ = o_ce.forward_backward(logits, targets)
    row0 = math.log(math.exp(2) + 1 + math.exp(-1)) - 2
    row1 = math.log(math.exp(0.5) + math.exp(1.5) + math.exp(-0.5)) + 0.5
    assert abs(loss.item() - 1.2887259920) < 1e-9
    assert abs(loss.item() - (row0 + row1) / 2) < 1e-12


@pytest.mark.parametrize("layout", ["2d", "3d"])
def test_cross_entropy_oracle_matches_torch_library(layout):
    torch.manual_seed(8)
    if layout == "2d":
        logits = 2 * torch.randn(40, 33, dtype=torch.float64)
        targets = torch.randint(0, 33, (40,))
        targets[::7] = -100
    else:
        logits = 2 * torch.randn(3, 33, 9, dtype=torch.float64)
        targets = torch.randint(0, 33, (3, 9))
        targets[0, ::4] = -100
    lr = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(lr, targets, ignore_index=-100)
    ref.backward()
    loss, grad = o_ce.forward_backward(logits, targets)
    torch.testing.assert_close(loss, ref.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(grad, lr.grad, rtol=1e-10, atol=1e-12)


def test_cross_entropy_oracle_invariants():
    v = 50
    logits = torch.zeros(4, v, dtype=torch.float64)
    targets = torch.tensor([1, -100, 3, 49])
    loss, grad = o_ce.forward_backward(logits, targets)
    assert abs(loss.item() - math.log(v)) < 1e-12  # uniform logits -> ln V
    torch.testing.assert_close(grad.sum(-1), torch.zeros(4, dtype=torch.float64))  # rows sum to 0
    assert torch.equal(grad[1], torch.zeros(v, dtype=torch.float64))  # ignored row is 0


def test_cross_entropy_fallback_restatement():
    torch.manual_seed(9)
    logits = (2 * torch.randn(16, 40)).bfloat16()
    targets = torch.randint(0, 40, (16,))
    targets[3] = -100
    loss, grad = o_ce.fallback_forward_backward(logits, targets)
    loss64, grad64 = o_ce.forward_backward(logits, targets)
    assert abs(loss.item() - loss64.item()) < 1e-5 * abs(loss64.item())
    torch.testing.assert_close(grad.double(), grad64, rtol=1e-5, atol=1e-8)


# ------------------------------------------------------------------ AdamW


def test_adamw_known_answer_reference_case():
    # reference tests/test_triton_ce_adamw.py:27-38: p=1, g=1, lr .1, betas (.9,.999),
    # eps 1e-8, wd .01 -> 0.899 after one step
    one = torch.tensor([1.0], dtype=torch.float64)
    p, m, v = o_adamw.step(one, one, 0 * one, 0 * one, t=1, lr=0.1, beta1=0.9, beta2=0.999,
                           eps=1e-8, weight_decay=0.01)
    assert abs(p.item() - 0.899) < 1e-8
    torch.testing.assert_close(m, 0.1 * one)
    torch.testing.assert_close(v, 0.001 * one)


def test_adamw_oracle_matches_torch_optimizer_over_steps():
    torch.manual_seed(10)
    p0 = 0.02 * torch.randn(1000, dtype=torch.float64)
    grads = [1e-3 * torch.randn(1000, dtype=torch.float64) for _ in range(4)]
    param = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([param], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                            foreach=False)
    p, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for t, g in enumerate(grads, start=1):
        param.grad = g.clone()
        opt.step()
        p, m, v = o_adamw.step(p, g, m, v, t=t, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                               weight_decay=0.1)
    torch.testing.assert_close(p, param.detach(), rtol=1e-12, atol=1e-15)
    torch.testing.assert_close(m, opt.state[param]["exp_avg"], rtol=1e-12, atol=1e-18)
    torch.testing.assert_close(v, opt.state[param]["exp_avg_sq"], rtol=1e-12, atol=1e-22)


def test_adamw_zero_gradient_no_decay_is_identity():
    p0 = torch.randn(10, dtype=torch.float64)
    z = torch.zeros(10, dtype=torch.float64)
    p, m, v = o_adamw.step(p0, z, z, z, t=1, lr=0.1, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.0)
    assert torch.equal(p, p0) and torch.equal(m, z) and torch.equal(v, z)


def test_cross_entropy_shifted_oracle_matches_torch_autograd_through_the_slice():
    # the train loop's exact expression, differentiated by torch through slice + transpose
    torch.manual_seed(10)
    b, s, v = 3, 7, 29
    logits = 2 * torch.randn(b, s, v, dtype=torch.float64)
    ids = torch.randint(0, v, (b, s))
    ids[1, 3] = -100
    ids[2, 0] = -100  # position 0 is never a target: must not matter
    lr = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(lr[:, :-1, :].transpose(1, 2), ids[:, 1:])
    ref.backward()
    loss, grad = o_ce.shifted_forward_backward(logits, ids)
    torch.testing.assert_close(loss, ref.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(grad, lr.grad, rtol=1e-10, atol=1e-12)
    assert torch.equal(grad[:, -1, :], torch.zeros(b, v, dtype=torch.float64))


@pytest.mark.parametrize("max_norm", [0.5, 1e6])
def test_clip_grad_norm_oracle_matches_torch_library(max_norm):
    torch.manual_seed(11)
    grads = [torch.randn(n, dtype=torch.float64) * s for n, s in ((7, 1.0), (300, 0.1), (1, 3.0))]
    params = [torch.nn.Parameter(torch.zeros_like(g)) for g in grads]
    for p, g in zip(params, grads):
        p.grad = g.clone()
    ref_total = torch.nn.utils.clip_grad_norm_(params, max_norm)
    total, clipped = o_adamw.clip_grad_norm(grads, max_norm)
    torch.testing.assert_close(total, ref_total, rtol=1e-12, atol=0)
    for c, p in zip(clipped, params):
        torch.testing.assert_close(c, p.grad, rtol=1e-12, atol=0)
    if max_norm > 1e3:  # below the norm: the coefficient clamps to exactly 1
        for c, g in zip(clipped, grads):
            assert torch.equal(c, g)


def test_residual_rmsnorm_oracle_matches_torch_autograd_of_the_block():
    # h = x + r feeds both the norm and a later residual add (out = h + mlp(norm(h)));
    # torch's autograd of that graph gives dx = dr = dh_in + d norm / d h
    torch.manual_seed(12)
    x = torch.randn(3, 5, 16, dtype=torch.float64, requires_grad=True)
    r = torch.randn(3, 5, 16, dtype=torch.float64, requires_grad=True)
    w = (1 + 0.02 * torch.randn(16, dtype=torch.float64)).requires_grad_(True)
    eps = 1e-5
    h = x + r
    y = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps) * w
    dy = torch.randn_like(y)
    dh_in = torch.randn_like(h)
    torch.autograd.backward([y, h], [dy, dh_in])
    oh, oy, _ = o_rms.residual_forward(x.detach(), r.detach(), w.detach(), eps)
    torch.testing.assert_close(oh, h.detach(), rtol=0, atol=0)
    torch.testing.assert_close(oy, y.detach(), rtol=1e-12, atol=1e-12)
    dh, dw = o_rms.residual_backward(dy, dh_in, oh, w.detach(), eps)
    torch.testing.assert_close(dh, x.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dh, r.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dw, w.grad, rtol=1e-10, atol=1e-12)


def test_residual_rmsnorm_oracle_rounds_h_like_torch():
    torch.manual_seed(13)
    x = torch.randn(64, 32).bfloat16()
    r = torch.randn(64, 32).bfloat16()
    h, _, _ = o_rms.residual_forward(x, r, torch.ones(32), 1e-6)
    assert h.dtype == torch.bfloat16
    assert torch.equal(h, x + r)  # torch's bf16 add: fp32 sum rounded once


def test_zero_unscale_and_check_oracle():
    g = [torch.tensor([1.5, -3.0, 2.0**-20]), torch.tensor([[7.0, 0.25]])]
    found, out = o_adamw.unscale_and_check(g, 1024.0)
    assert not found
    for a, b in zip(out, g):
        assert torch.equal(a, b / 1024)  # a power-of-two scale divides exactly
    bad = [g[0], torch.tensor([1.0, float("nan")])]
    found, out = o_adamw.unscale_and_check(bad, 1024.0)
    assert found and all(x is y for x, y in zip(out, bad))  # untouched
    found, _ = o_adamw.unscale_and_check([torch.tensor([float("-inf")])], 2.0)
    assert found


@pytest.mark.parametrize("max_norm", [0.5, 1e3])
def test_zero_clip_oracle_matches_torch_clip_when_clipping(max_norm):
    torch.manual_seed(14)
    grads = [torch.randn(n, dtype=torch.float64) for n in (10, 100)]
    total, out = o_adamw.zero_clip_grad_norm(grads, max_norm)
    params = [torch.nn.Parameter(torch.zeros_like(g)) for g in grads]
    for p, g in zip(params, grads):
        p.grad = g.clone()
    ref_total = torch.nn.utils.clip_grad_norm_(params, max_norm)
    torch.testing.assert_close(total, ref_total, rtol=1e-12, atol=0)
    for o, p, g in zip(out, params, grads):
        if max_norm < 1:  # coefficient below 1: both clip the same way
            torch.testing.assert_close(o, p.grad, rtol=1e-12, atol=0)
        else:  # no clipping at all (torch multiplies by exactly 1)
            assert torch.equal(o, g) and torch.equal(p.grad, g)
