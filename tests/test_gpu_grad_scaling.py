"""Loss-scaling and ZeRO gradient handling (unscale + finite check, ZeRO clip, and the
fused unscale + clip + AdamW step) against the oracle and torch, through the C ABI."""

from __future__ import annotations

import pytest
import torch

from gpu_util import close_fp32, randn
from oracle import adamw as o_adamw
from picotron_amd.nn.triton_kernels import (
    triton_unscale_and_check_,
    triton_unscale_clip_and_step,
    triton_zero_clip_grad_norm_,
)

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SIZES = [1, 3, 4095, 4096, 4097, 70_000, 1 << 20]


def _params(gpu, seed, scale=1.0, sizes=SIZES):
    ps = [torch.nn.Parameter(randn((n,), torch.float32, gpu, seed + n, 0.02)) for n in sizes]
    for i, p in enumerate(ps):
        p.grad = randn(p.shape, torch.float32, gpu, seed + 1000 + i, 1e-3 * scale)
    return ps


@pytest.mark.parametrize("scale", [65536.0, 3000.0])
def test_unscale_and_check_finite(gpu, scale):
    ps = _params(gpu, 1, scale)
    grads = [p.grad.clone() for p in ps]
    assert triton_unscale_and_check_(ps, scale) is False
    found, ref = o_adamw.unscale_and_check(grads, scale)
    assert not found
    for p, r in zip(ps, ref):
        assert torch.equal(p.grad, r)  # the same fp32 multiply by fp32(1/scale), bit for bit


@pytest.mark.parametrize("bad", [float("inf"), float("-inf"), float("nan")])
def test_unscale_and_check_non_finite_leaves_everything(gpu, bad):
    ps = _params(gpu, 2, 1024.0)
    ps[4].grad[4096] = bad  # the second block of one tensor
    grads = [p.grad.clone() for p in ps]
    assert triton_unscale_and_check_(ps, 1024.0) is True
    for p, g in zip(ps, grads):
        assert torch.equal(p.grad.nan_to_num(), g.nan_to_num())


@pytest.mark.parametrize("max_norm", [0.05, 1e4])
def test_zero_clip(gpu, max_norm):
    ps = _params(gpu, 3)
    grads = [p.grad.clone() for p in ps]
    total = triton_zero_clip_grad_norm_(ps, max_norm)
    ref_total, ref = o_adamw.zero_clip_grad_norm(grads, max_norm)
    assert abs(total.item() - ref_total.item()) <= 1e-6 * ref_total.item()
    for p, r, g in zip(ps, ref, grads):
        if max_norm > 1e3:
            assert torch.equal(p.grad, g)  # coefficient >= 1: no pass over the gradients
        else:
            close_fp32(p.grad, r)


@pytest.mark.parametrize("max_norm", [None, 0.05, 1e4])
def test_fused_unscale_clip_step_matches_the_reference_sequence(gpu, max_norm):
    scale = 32768.0
    fused = _params(gpu, 4, scale)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    for a, b in zip(fused, ref):
        b.grad = a.grad.clone()
    opt_f = torch.optim.AdamW(fused, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    for step in range(2):
        if step:
            for i, (a, b) in enumerate(zip(fused, ref)):
                g = randn(a.shape, torch.float32, gpu, 77 + i, 1e-3 * scale)
                a.grad, b.grad = g, g.clone()
        # reference: unscale_and_check_ -> clip_grad_norm_ (ZeRO semantics) -> step
        found, unscaled = o_adamw.unscale_and_check([b.grad for b in ref], scale)
        assert not found
        if max_norm is not None:
            _, clipped = o_adamw.zero_clip_grad_norm(unscaled, max_norm, compute=torch.float32)
        else:
            clipped = unscaled
        for b, g in zip(ref, clipped):
            b.grad = g
        opt_r.step()
        assert triton_unscale_clip_and_step(opt_f, scale, max_norm) is False
        for a, b in zip(fused, ref):
            close_fp32(a.grad, b.grad)  # left unscaled and clipped, as the reference leaves them
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        close_fp32(opt_f.state[a]["exp_avg"], opt_r.state[b]["exp_avg"])
        close_fp32(opt_f.state[a]["exp_avg_sq"], opt_r.state[b]["exp_avg_sq"])


def test_fused_step_skips_on_overflow_and_rescales_unowned(gpu):
    owned = _params(gpu, 5, 1024.0, sizes=[5000, 17])
    extra = _params(gpu, 6, 1024.0, sizes=[300])
    opt = torch.optim.AdamW(owned, **HP)
    before = [p.detach().clone() for p in owned]
    grads = [p.grad.clone() for p in owned + extra]
    extra[0].grad[7] = float("nan")
    assert triton_unscale_clip_and_step(opt, 1024.0, 1.0, parameters=owned + extra) is True
    assert len(opt.state) == 0  # no state created, no step counted
    for p, b in zip(owned, before):
        assert torch.equal(p.detach(), b)
    for p, g in zip(owned, grads):
        assert torch.equal(p.grad, g)
    extra[0].grad[7] = 0.0
    g_extra = extra[0].grad.clone()
    assert triton_unscale_clip_and_step(opt, 1024.0, None, parameters=owned + extra) is False
    assert torch.equal(extra[0].grad, g_extra * (1.0 / 1024.0))  # not stepped, but unscaled
    assert float(opt.state[owned[0]]["step"]) == 1.0
    # an overflow on a later step: the existing state stays as it was, the counter included
    moments = [(opt.state[p]["exp_avg"].clone(), opt.state[p]["exp_avg_sq"].clone()) for p in owned]
    after_first = [p.detach().clone() for p in owned]
    owned[1].grad[3] = float("inf")
    assert triton_unscale_clip_and_step(opt, 1024.0, 1.0, parameters=owned + extra) is True
    for p, b, (m, v) in zip(owned, after_first, moments):
        assert float(opt.state[p]["step"]) == 1.0
        assert torch.equal(p.detach(), b)
        assert torch.equal(opt.state[p]["exp_avg"], m) and torch.equal(opt.state[p]["exp_avg_sq"], v)
