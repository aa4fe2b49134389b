"""Fused AdamW parity of the HIP kernel (through the C ABI) with the oracle and torch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import close_fp32, from_npz, randn
from oracle import adamw as o_adamw
from picotron_amd import ops
from picotron_amd.nn.triton_kernels import AdamWStepWithFallback, triton_adamw_step

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def test_reference_known_answer(gpu):
    p = torch.nn.Parameter(torch.tensor([1.0], device=gpu))
    opt = torch.optim.AdamW([p], lr=0.1, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    p.grad = torch.tensor([1.0], device=gpu)
    triton_adamw_step(opt)
    assert abs(p.item() - 0.899) < 1e-6
    assert float(opt.state[p]["step"]) == 1.0


def test_golden_fixture(gpu):
    f = np.load(GOLDEN / "adamw_small.npz")
    sizes = [int(n) for n in f["sizes"]]
    params = [torch.nn.Parameter(from_npz(f[f"p0_{i}"], gpu)) for i in range(len(sizes))]
    opt = torch.optim.AdamW(params, **HP)
    for t in range(1, int(f["steps"]) + 1):
        for i, p in enumerate(params):
            p.grad = from_npz(f[f"g{t}_{i}"], gpu)
        triton_adamw_step(opt)
    for i, p in enumerate(params):
        close_fp32(p.detach(), from_npz(f[f"p_{i}"], gpu))
        close_fp32(opt.state[p]["exp_avg"], from_npz(f[f"m_{i}"], gpu))
        close_fp32(opt.state[p]["exp_avg_sq"], from_npz(f[f"v_{i}"], gpu))


def test_matches_torch_adamw_multi_tensor(gpu):
    sizes = [1, 3, 4095, 4096, 4097, 70_000, 1 << 20]
    fused = [torch.nn.Parameter(randn((n,), torch.float32, gpu, n, 0.02)) for n in sizes]
    fused.append(torch.nn.Parameter(randn((33, 65), torch.float32, gpu, 5, 0.02)))
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    opt_f = torch.optim.AdamW(fused, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    for step in range(4):
        for i, (a, b) in enumerate(zip(fused, ref)):
            g = randn(a.shape, torch.float32, gpu, 100 * step + i, 1e-3)
            a.grad, b.grad = g, g.clone()
        for group in (opt_f.param_groups[0], opt_r.param_groups[0]):
            group["lr"] = 3e-4 * (1 + step)  # the train loop rewrites lr every step
        triton_adamw_step(opt_f)
        opt_r.step()
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        close_fp32(opt_f.state[a]["exp_avg"], opt_r.state[b]["exp_avg"])
        close_fp32(opt_f.state[a]["exp_avg_sq"], opt_r.state[b]["exp_avg_sq"])
    # the state dict has torch's layout and loads into a torch AdamW
    sd = opt_f.state_dict()
    opt_r.load_state_dict(sd)
    assert set(sd["state"][0]) == {"step", "exp_avg", "exp_avg_sq"}
    assert sd["state"][0]["step"].device.type == "cpu" and float(sd["state"][0]["step"]) == 4.0


def _many_sizes(count: int, seed: int) -> list[int]:
    """Sizes that put record boundaries everywhere: single elements, exactly one 1024-element
    block, one block and one element, and larger tensors, shuffled."""

    rng = np.random.default_rng(seed)
    base = [1, 2, 1023, 1024, 1025, 2048, 4096, 5000, 65_536, 300_001]
    return [int(x) for x in rng.permutation(np.resize(base, count))]


@pytest.mark.parametrize("count", [17, 300, 1500])
def test_many_tensors_find_their_blocks(gpu, count):
    """One launch over hundreds of tensors: every block must find its own record (a search
    over the table of several rounds), for the step and for the fused clip's walks."""

    from picotron_amd.nn.triton_kernels import triton_clip_grad_norm_and_step

    sizes = _many_sizes(count, count)
    print(f"many tensors: {count} records, {sum(sizes)} elements", flush=True)
    fused = [torch.nn.Parameter(randn((n,), torch.float32, gpu, 7 * i, 0.02)) for i, n in enumerate(sizes)]
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    opt_f = torch.optim.AdamW(fused, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    for step in range(2):
        for i, (a, b) in enumerate(zip(fused, ref)):
            g = randn(a.shape, torch.float32, gpu, 1000 * step + i, 1e-3)
            a.grad, b.grad = g, g.clone()
        if step == 0:
            triton_adamw_step(opt_f)
        else:
            ref_total = torch.nn.utils.clip_grad_norm_(ref, 0.05)
            total = triton_clip_grad_norm_and_step(opt_f, 0.05)
            close_fp32(total.reshape(()), ref_total.reshape(()))
        opt_r.step()
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        close_fp32(a.grad, b.grad)
        close_fp32(opt_f.state[a]["exp_avg"], opt_r.state[b]["exp_avg"])
        close_fp32(opt_f.state[a]["exp_avg_sq"], opt_r.state[b]["exp_avg_sq"])


def test_many_tensors_zero_clip_scales_every_gradient(gpu):
    """The ZeRO clip's in-place scaling walk over 300 tensors: every gradient scaled once."""

    from picotron_amd.nn.triton_kernels import triton_zero_clip_grad_norm_

    sizes = _many_sizes(300, 5)
    params = [torch.nn.Parameter(torch.zeros(n, device=gpu)) for n in sizes]
    grads = [randn((n,), torch.float32, gpu, 3 * i + 1, 1e-3) for i, n in enumerate(sizes)]
    for p, g in zip(params, grads):
        p.grad = g.clone()
    norm = torch.linalg.vector_norm(torch.cat([g.double() for g in grads]))
    total = triton_zero_clip_grad_norm_(params, 0.01)
    close_fp32(total.double().reshape(()), norm)
    coef = 0.01 / (float(total) + 1e-6)
    for p, g in zip(params, grads):
        close_fp32(p.grad, g * coef)


def test_param_groups_late_group_and_fused_clip(gpu):
    # Several groups with their own hyperparameters, a group added after two steps (its
    # parameters count their own steps: one launch per distinct step value), a parameter
    # without a gradient, and the clip's norm taken over every group, against torch
    def make(seed_base):
        decay = [torch.nn.Parameter(randn((300, 17), torch.float32, gpu, seed_base + 1, 0.02)),
                 torch.nn.Parameter(randn((4096,), torch.float32, gpu, seed_base + 2, 0.02))]
        no_decay = [torch.nn.Parameter(randn((4096,), torch.float32, gpu, seed_base + 3, 0.02)),
                    torch.nn.Parameter(randn((5,), torch.float32, gpu, seed_base + 4, 0.02))]
        late = [torch.nn.Parameter(randn((777,), torch.float32, gpu, seed_base + 5, 0.02))]
        return decay, no_decay, late

    fused, ref = make(0), make(0)
    groups = lambda ps: [dict(params=ps[0], lr=1e-3, weight_decay=0.1),
                         dict(params=ps[1], lr=5e-4, weight_decay=0.0, betas=(0.8, 0.9), eps=1e-6)]
    opt_f = torch.optim.AdamW(groups(fused), betas=(0.9, 0.95), eps=1e-8)
    opt_r = torch.optim.AdamW(groups(ref), betas=(0.9, 0.95), eps=1e-8, foreach=False)
    stepper = AdamWStepWithFallback(use_triton=True)
    for step in range(4):
        if step == 2:
            opt_f.add_param_group(dict(params=fused[2], lr=2e-3, weight_decay=0.05))
            opt_r.add_param_group(dict(params=ref[2], lr=2e-3, weight_decay=0.05))
        for gi, (gf, gr) in enumerate(zip(fused, ref)):
            for pi, (a, b) in enumerate(zip(gf, gr)):
                if gi == 1 and pi == 1 and step == 1:
                    a.grad = b.grad = None  # skipped this step
                    continue
                g = randn(a.shape, torch.float32, gpu, 1000 * step + 10 * gi + pi, 0.05)
                a.grad, b.grad = g, g.clone()
        stepper.step(opt_f, max_grad_norm=1.0)
        params_r = [p for ps in (ref if step >= 2 else ref[:2]) for p in ps]
        torch.nn.utils.clip_grad_norm_(params_r, 1.0)
        opt_r.step()
    assert not stepper._fallback_warned
    for gf, gr in zip(fused, ref):
        for a, b in zip(gf, gr):
            close_fp32(a.detach(), b.detach())
            sa, sb = opt_f.state[a], opt_r.state[b]
            assert float(sa["step"]) == float(sb["step"])
            close_fp32(sa["exp_avg"], sb["exp_avg"])
            close_fp32(sa["exp_avg_sq"], sb["exp_avg_sq"])
    assert float(opt_f.state[fused[2][0]]["step"]) == 2.0 and float(opt_f.state[fused[1][1]]["step"]) == 3.0


@pytest.mark.parametrize(
    "options",
    [dict(amsgrad=True), dict(maximize=True), dict(lr=torch.tensor(1e-3)), dict(fused=True)],
    ids=["amsgrad", "maximize", "tensor_lr", "torch_fused"],
)
def test_unsupported_options_fall_back_to_torch(gpu, options):
    # Options the fused step does not implement: the step raises TritonAdamWUnavailable
    # before touching any state, AdamWStepWithFallback warns once and runs torch's own
    # step, and the result equals torch's
    import warnings

    from picotron_amd.nn.triton_kernels import TritonAdamWUnavailable

    hp = dict(HP, **options)
    if "lr" in options:
        hp["lr"] = torch.tensor(1e-3)
    fused = [torch.nn.Parameter(randn((1000,), torch.float32, gpu, 1, 0.02))]
    ref = [torch.nn.Parameter(fused[0].detach().clone())]
    opt_f, opt_r = torch.optim.AdamW(fused, **hp), torch.optim.AdamW(ref, **hp)
    g = randn((1000,), torch.float32, gpu, 2, 1e-3)
    fused[0].grad, ref[0].grad = g, g.clone()
    with pytest.raises(TritonAdamWUnavailable, match="not implemented"):
        triton_adamw_step(opt_f)
    assert len(opt_f.state) == 0  # nothing touched
    stepper = AdamWStepWithFallback(use_triton=True)
    with warnings.catch_warnings(record=True) as records:
        warnings.simplefilter("always")
        stepper.step(opt_f)
        stepper.step(opt_f)
    assert sum("Triton AdamW unavailable" in str(w.message) for w in records) == 1
    opt_r.step()
    opt_r.step()
    assert torch.equal(fused[0].detach(), ref[0].detach())


def test_checkpoint_round_trip_continues_identically(gpu):
    # picotron saves and restores optimizer.state_dict() (src/picotron/serialize/checkpoint.py:
    # 50,91): a torch-written state resumes under the fused step, and a fused-written state
    # resumes under torch's step, each continuing as the other would
    import copy

    sizes = [(513, 7), (1000,), (1,)]

    def grads(step):
        return [randn(sz, torch.float32, gpu, 40 * step + i, 1e-3) for i, sz in enumerate(sizes)]

    torch_params = [torch.nn.Parameter(randn(sz, torch.float32, gpu, i, 0.02)) for i, sz in enumerate(sizes)]
    torch_opt = torch.optim.AdamW(torch_params, foreach=False, **HP)
    for step in range(2):
        for p, g in zip(torch_params, grads(step)):
            p.grad = g
        torch_opt.step()
    fused_params = [torch.nn.Parameter(p.detach().clone()) for p in torch_params]
    fused_opt = torch.optim.AdamW(fused_params, **HP)
    fused_opt.load_state_dict(copy.deepcopy(torch_opt.state_dict()))
    for step in (2, 3):
        for a, b, g in zip(fused_params, torch_params, grads(step)):
            a.grad, b.grad = g, g.clone()
        triton_adamw_step(fused_opt)
        torch_opt.step()
    # and back: the fused optimizer's state into a fresh torch optimizer
    resumed = [torch.nn.Parameter(p.detach().clone()) for p in fused_params]
    resumed_opt = torch.optim.AdamW(resumed, foreach=False, **HP)
    resumed_opt.load_state_dict(copy.deepcopy(fused_opt.state_dict()))
    for a, b, g in zip(resumed, torch_params, grads(4)):
        a.grad, b.grad = g, g.clone()
    resumed_opt.step()
    torch_opt.step()
    for a, b in zip(resumed, torch_params):
        close_fp32(a.detach(), b.detach())
        sa, sb = resumed_opt.state[a], torch_opt.state[b]
        assert float(sa["step"]) == float(sb["step"]) == 5.0
        close_fp32(sa["exp_avg"], sb["exp_avg"])
        close_fp32(sa["exp_avg_sq"], sb["exp_avg_sq"])


def test_new_moments_share_one_allocation_and_save_like_torch(gpu):
    """The fused step creates a group's moments as aligned, contiguous views of one allocation
    (each with its parameter's shape); torch.save / torch.load of the state dict, as picotron's
    checkpoint writes it (src/picotron/serialize/checkpoint.py:50), brings them back into a
    torch optimizer that continues as the fused one does."""

    import io

    sizes = [(513, 7), (0,), (1000,), (1,), (64, 3)]
    params = [torch.nn.Parameter(randn(sz, torch.float32, gpu, 50 + i, 0.02)) for i, sz in enumerate(sizes)]
    opt = torch.optim.AdamW(params, **HP)
    for p in params:
        p.grad = randn(p.shape, torch.float32, gpu, 60 + p.numel(), 1e-3)
    triton_adamw_step(opt)
    moments = [opt.state[p][k] for p in params for k in ("exp_avg", "exp_avg_sq")]
    base = moments[0].untyped_storage().data_ptr()
    for p in params:
        for k in ("exp_avg", "exp_avg_sq"):
            m = opt.state[p][k]
            assert m.shape == p.shape and m.is_contiguous() and m.dtype == torch.float32
            assert m.untyped_storage().data_ptr() == base
            assert m.numel() == 0 or m.data_ptr() % 256 == 0
    # no two moments overlap
    spans = sorted((m.data_ptr(), m.data_ptr() + 4 * m.numel()) for m in moments if m.numel())
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))

    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    loaded = torch.load(buf, map_location=gpu, weights_only=True)
    resumed = [torch.nn.Parameter(p.detach().clone()) for p in params]
    resumed_opt = torch.optim.AdamW(resumed, foreach=False, **HP)
    resumed_opt.load_state_dict(loaded)
    for a, b in zip(params, resumed):
        a.grad = randn(a.shape, torch.float32, gpu, 70 + a.numel(), 1e-3)
        b.grad = a.grad.clone()
    triton_adamw_step(opt)
    resumed_opt.step()
    for a, b in zip(params, resumed):
        close_fp32(a.detach(), b.detach())
        close_fp32(opt.state[a]["exp_avg"], resumed_opt.state[b]["exp_avg"])
        close_fp32(opt.state[a]["exp_avg_sq"], resumed_opt.state[b]["exp_avg_sq"])
        assert float(opt.state[a]["step"]) == float(resumed_opt.state[b]["step"]) == 2.0


def test_unaligned_views_and_missing_grads(gpu):
    flat = randn((10_001,), torch.float32, gpu, 9, 0.02)
    params = [torch.nn.Parameter(flat[1:5000].clone()), torch.nn.Parameter(flat[:7].clone())]
    ref = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt_f = torch.optim.AdamW(params, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    g = randn((6000,), torch.float32, gpu, 10, 1e-3)
    params[0].grad, ref[0].grad = g[1:5000], g[1:5000].clone()  # 4-byte-offset gradient
    triton_adamw_step(opt_f)
    opt_r.step()
    close_fp32(params[0].detach(), ref[0].detach())
    assert torch.equal(params[1].detach(), ref[1].detach())  # no grad: untouched
    assert len(opt_f.state[params[1]]) == 0


def test_full_config(gpu):
    # one step over 1.2e9 fp32 params ~ N(0, 0.02^2), grads ~ N(0, 1e-3^2), at step 2
    n = 1_200_000_000
    p = torch.nn.Parameter(randn((n,), torch.float32, gpu, 91, 0.02))
    opt = torch.optim.AdamW([p], **HP)
    p.grad = randn((n,), torch.float32, gpu, 92, 1e-3)
    step = AdamWStepWithFallback(use_triton=True)
    step.step(opt)  # step 1 creates the state
    m1 = opt.state[p]["exp_avg"].clone()
    v1 = opt.state[p]["exp_avg_sq"].clone()
    p1 = p.detach().clone()
    p.grad = randn((n,), torch.float32, gpu, 93, 1e-3)
    step.step(opt)
    assert not step._fallback_warned
    # fp32 oracle evaluated by torch on the GPU, in slices (memory)
    for lo in range(0, n, 200_000_000):
        hi = min(n, lo + 200_000_000)
        ep, em, ev = o_adamw.step(
            p1[lo:hi], p.grad[lo:hi], m1[lo:hi], v1[lo:hi], t=2, lr=3e-4, beta1=0.9, beta2=0.95,
            eps=1e-8, weight_decay=0.1, compute=torch.float32,
        )
        close_fp32(p.detach()[lo:hi], ep)
        close_fp32(opt.state[p]["exp_avg"][lo:hi], em)
        close_fp32(opt.state[p]["exp_avg_sq"][lo:hi], ev)


def _clip_pair(gpu, sizes, seed):
    fused = [torch.nn.Parameter(randn((n,), torch.float32, gpu, seed + n, 0.02)) for n in sizes]
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    return fused, ref


@pytest.mark.parametrize("max_norm", [0.05, 1e4])
def test_clip_grad_norm_and_step_matches_torch(gpu, max_norm):
    # torch.nn.utils.clip_grad_norm_ then torch AdamW (the reference train loop) against the
    # fused clip + step: clipping active (norm ~ 1.3) and inactive (coefficient exactly 1)
    from picotron_amd.nn.triton_kernels import triton_clip_grad_norm_and_step

    sizes = [1, 3, 4095, 4096, 4097, 70_000, 1 << 20]
    fused, ref = _clip_pair(gpu, sizes, 7)
    opt_f = torch.optim.AdamW(fused, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    for step in range(3):
        for i, (a, b) in enumerate(zip(fused, ref)):
            g = randn(a.shape, torch.float32, gpu, 50 * step + i, 1e-3)
            a.grad, b.grad = g, g.clone()
        ref_total = torch.nn.utils.clip_grad_norm_(ref, max_norm)
        opt_r.step()
        total = triton_clip_grad_norm_and_step(opt_f, max_norm)
        close_fp32(total.reshape(()), ref_total.reshape(()))
        for a, b in zip(fused, ref):
            close_fp32(a.grad, b.grad)  # left clipped, as clip_grad_norm_ leaves them
            if max_norm > 1e3:
                assert torch.equal(a.grad, b.grad)
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        close_fp32(opt_f.state[a]["exp_avg"], opt_r.state[b]["exp_avg"])
        close_fp32(opt_f.state[a]["exp_avg_sq"], opt_r.state[b]["exp_avg_sq"])


def test_clip_without_write_back_and_the_oracle(gpu):
    from picotron_amd.nn.triton_kernels import triton_clip_grad_norm_and_step

    sizes = [5000, 123, 4096 * 3]
    fused, _ = _clip_pair(gpu, sizes, 9)
    grads = [randn(p.shape, torch.float32, gpu, 900 + i, 0.05) for i, p in enumerate(fused)]
    for p, g in zip(fused, grads):
        p.grad = g.clone()
    p0 = [p.detach().clone() for p in fused]
    opt = torch.optim.AdamW(fused, **HP)
    total = triton_clip_grad_norm_and_step(opt, 0.5, write_back_grads=False)
    ref_total, clipped = o_adamw.clip_grad_norm(grads, 0.5)
    assert abs(total.item() - ref_total.item()) <= 1e-6 * ref_total.item()
    for p, g, c, q in zip(fused, grads, clipped, p0):
        assert torch.equal(p.grad, g)  # gradients keep their unclipped values
        ep, _, _ = o_adamw.step(q, c, torch.zeros_like(q), torch.zeros_like(q), t=1, lr=HP["lr"],
                                beta1=HP["betas"][0], beta2=HP["betas"][1], eps=HP["eps"],
                                weight_decay=HP["weight_decay"])
        close_fp32(p.detach(), ep.float())


def test_clip_non_finite_gradients_propagate_like_torch(gpu):
    from picotron_amd.nn.triton_kernels import triton_clip_grad_norm_and_step

    fused, ref = _clip_pair(gpu, [4096, 10], 11)
    for a, b in zip(fused, ref):
        g = randn(a.shape, torch.float32, gpu, 3, 1e-3)
        a.grad, b.grad = g, g.clone()
    fused[1].grad[3] = float("inf")
    ref[1].grad[3] = float("inf")
    ref_total = torch.nn.utils.clip_grad_norm_(ref, 1.0)
    torch.optim.AdamW(ref, foreach=False, **HP).step()
    total = triton_clip_grad_norm_and_step(torch.optim.AdamW(fused, **HP), 1.0)
    assert torch.isinf(total) and torch.isinf(ref_total)
    for a, b in zip(fused, ref):
        assert torch.equal(torch.isnan(a.detach()), torch.isnan(b.detach()))
        assert torch.equal(torch.isnan(a.grad), torch.isnan(b.grad))


def test_stepper_with_clipping_and_no_gradients(gpu):
    from picotron_amd.nn.triton_kernels import triton_clip_grad_norm_and_step

    p = torch.nn.Parameter(torch.ones(8, device=gpu))
    opt = torch.optim.AdamW([p], **HP)
    assert float(triton_clip_grad_norm_and_step(opt, 1.0)) == 0.0  # nothing has a gradient
    assert len(opt.state) == 0
    fused, ref = _clip_pair(gpu, [300], 13)
    fused[0].grad = torch.full_like(fused[0], 2.0)
    ref[0].grad = torch.full_like(ref[0], 2.0)
    stepper = AdamWStepWithFallback(use_triton=True)
    stepper.step(torch.optim.AdamW(fused, **HP), max_grad_norm=1.0)
    assert not stepper._fallback_warned
    torch.nn.utils.clip_grad_norm_(ref, 1.0)
    torch.optim.AdamW(ref, foreach=False, **HP).step()
    close_fp32(fused[0].detach(), ref[0].detach())


@pytest.mark.parametrize(
    "bad",
    ["short", "offloaded", "float64", "strided", "no_moment"],
)
def test_mismatched_resumed_state_is_refused_before_launch(gpu, bad):
    """A state loaded from a checkpoint that does not match the parameter (short, on the CPU,
    fp64, a strided view, missing a moment) is refused by the fused step with nothing
    launched and nothing changed; torch's own step decides what happens then."""

    p = torch.nn.Parameter(randn((5000,), torch.float32, gpu, 3))
    p.grad = randn((5000,), torch.float32, gpu, 4)
    opt = torch.optim.AdamW([p], **HP)
    m = torch.zeros(5000, device=gpu)
    states = {
        "short": dict(exp_avg=torch.zeros(4096, device=gpu), exp_avg_sq=m.clone()),
        "offloaded": dict(exp_avg=torch.zeros(5000), exp_avg_sq=m.clone()),
        "float64": dict(exp_avg=torch.zeros(5000, dtype=torch.float64, device=gpu), exp_avg_sq=m.clone()),
        "strided": dict(exp_avg=torch.zeros(10000, device=gpu)[::2], exp_avg_sq=m.clone()),
        "no_moment": dict(exp_avg_sq=m.clone()),
    }
    opt.state[p] = dict(step=torch.tensor(2.0), **states[bad])
    before = p.detach().clone()
    from picotron_amd.nn.triton_kernels import TritonAdamWUnavailable

    with pytest.raises(TritonAdamWUnavailable):
        triton_adamw_step(opt)
    torch.cuda.synchronize()
    assert torch.equal(p.detach(), before)
    assert float(opt.state[p]["step"]) == 2.0
