"""The train loop's single-GPU fp16 update (torch.amp.GradScaler: unscale_, clip_grad_norm_,
step, update; reference src/picotron/training/train_loop.py:155-160) fused, against the same
torch sequence step by step: parameters, moments, step counts, the scaler's scale and growth
tracker, and the gradients it leaves, over steps that grow the scale and steps that overflow."""

from __future__ import annotations

import warnings

import pytest
import torch

from gpu_util import close_fp32, randn
from picotron_amd.nn.triton_kernels import (
    AdamWStepWithFallback,
    TritonAdamWUnavailable,
    triton_grad_scaler_step,
)

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SIZES = [1, 3, 4095, 4096, 4097, 70_000, 1 << 20]


def _setup(gpu, seed):
    fused = [torch.nn.Parameter(randn((n,), torch.float32, gpu, seed + n, 0.02)) for n in SIZES]
    fused.append(torch.nn.Parameter(torch.ones(5, device=gpu)))  # never gets a gradient
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    opt_f = torch.optim.AdamW(fused, **HP)
    opt_r = torch.optim.AdamW(ref, foreach=False, **HP)
    scalers = []
    for _ in range(2):
        sc = torch.amp.GradScaler("cuda", init_scale=2.0 ** 16, growth_interval=2)
        sc.scale(torch.ones((), device=gpu))  # creates the scale tensor, as scale(loss) does
        scalers.append(sc)
    return fused, ref, opt_f, opt_r, scalers[0], scalers[1]


def _set_grads(fused, ref, gpu, seed, scale, bad=None):
    for i, (a, b) in enumerate(zip(fused[:-1], ref[:-1])):
        g = randn(a.shape, torch.float32, gpu, seed + i, 1e-3 * scale)
        if bad is not None and i == 4:
            g[4096] = bad  # the second block of one tensor
        a.grad, b.grad = g, g.clone()


def _reference_step(sc, opt, params, max_norm):
    sc.unscale_(opt)
    if max_norm is not None:
        torch.nn.utils.clip_grad_norm_(params, max_norm)
    sc.step(opt)
    sc.update()


def _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too):
    assert sc_f.get_scale() == sc_r.get_scale()
    assert sc_f._growth_tracker.item() == sc_r._growth_tracker.item()
    for a, b in zip(fused, ref):
        sa, sb = opt_f.state.get(a, {}), opt_r.state.get(b, {})
        assert set(sa) == set(sb)
        close_fp32(a.detach(), b.detach())
        if sb:
            assert sa["step"].item() == sb["step"].item()
            close_fp32(sa["exp_avg"], sb["exp_avg"])
            close_fp32(sa["exp_avg_sq"], sb["exp_avg_sq"])
        if grads_too and b.grad is not None:
            if torch.isfinite(b.grad).all():
                close_fp32(a.grad, b.grad)
            else:  # an overflow step without clipping: both are g * (1 / scale), exactly
                assert torch.equal(a.grad.nan_to_num(), b.grad.nan_to_num())


# (step, bad value): an overflow on the first step (no state may be created), one after the
# scale has grown, and a NaN right after a backoff
OVERFLOWS = {0: float("inf"), 3: float("-inf"), 4: float("nan")}


@pytest.mark.parametrize("max_norm", [None, 1e-3, 1e4])
def test_fused_grad_scaler_step_matches_torch_sequence(gpu, max_norm):
    fused, ref, opt_f, opt_r, sc_f, sc_r = _setup(gpu, 5)
    for step in range(8):
        scale = sc_r.get_scale()
        bad = OVERFLOWS.get(step)
        print(f"grad scaler step {step} scale {scale} bad {bad} max_norm {max_norm}", flush=True)
        _set_grads(fused, ref, gpu, 100 * step, scale, bad)
        _reference_step(sc_r, opt_r, ref, max_norm)
        skipped = triton_grad_scaler_step(sc_f, opt_f, max_norm)
        assert skipped == (bad is not None)
        # after a skipped step torch's clip has run on non-finite gradients (0 or NaN
        # everywhere); the fused path leaves them unscaled, as unscale_ does
        _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too=bad is None or max_norm is None)
    # the scale grew twice and backed off three times: 2^16 * 2^2 / 2^3
    assert sc_f.get_scale() == 2.0 ** 15


def test_unclipped_gradients_are_torch_bits(gpu):
    """With a power-of-two scale and no clipping the unscaled gradients are bitwise torch's."""

    fused, ref, opt_f, opt_r, sc_f, sc_r = _setup(gpu, 6)
    _set_grads(fused, ref, gpu, 7, sc_r.get_scale())
    _reference_step(sc_r, opt_r, ref, None)
    triton_grad_scaler_step(sc_f, opt_f, None)
    for a, b in zip(fused[:-1], ref[:-1]):
        assert torch.equal(a.grad, b.grad)


def test_fallback_class_uses_the_fused_path_without_warning(gpu):
    fused, ref, opt_f, opt_r, sc_f, sc_r = _setup(gpu, 7)
    stepper = AdamWStepWithFallback(use_triton=True)
    for step in range(3):
        scale = sc_r.get_scale()
        _set_grads(fused, ref, gpu, 300 + step, scale, float("inf") if step == 1 else None)
        _reference_step(sc_r, opt_r, ref, 1.0)
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            stepper.step_with_grad_scaler(sc_f, opt_f, 1.0)
        _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too=step != 1)


def test_already_unscaled_optimizer_is_rejected_untouched(gpu):
    """A caller that ran unscale_ itself is refused before anything changes (the fused path
    would unscale twice), so torch's own step() and update() can follow."""

    fused, ref, opt_f, opt_r, sc_f, sc_r = _setup(gpu, 8)
    _set_grads(fused, ref, gpu, 9, sc_r.get_scale())
    sc_f.unscale_(opt_f)
    grads = [p.grad.clone() for p in fused[:-1]]
    with pytest.raises(TritonAdamWUnavailable, match="already unscaled"):
        triton_grad_scaler_step(sc_f, opt_f, None)
    for p, g in zip(fused[:-1], grads):
        assert torch.equal(p.grad, g)
    assert not opt_f.state
    sc_f.step(opt_f)
    sc_f.update()
    _reference_step(sc_r, opt_r, ref, None)
    _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too=True)


def test_a_failure_after_the_update_began_is_not_retried_by_the_fallback(gpu, monkeypatch):
    # A launch error inside the fused update (here forced from the host by replacing the step
    # launcher) comes after the step counters were advanced and the gradients unscaled:
    # running torch's unscale_ / step again would unscale twice and count the step twice, so
    # the error propagates and nothing is applied a second time.
    from picotron_amd import _lib, ops
    from picotron_amd.nn.triton_kernels import FusedAdamWStepFailed

    fused, _, opt_f, _, sc_f, _ = _setup(gpu, 300)
    _set_grads(fused, fused, gpu, 301, sc_f.get_scale())
    hook = AdamWStepWithFallback(use_triton=True)
    hook.step_with_grad_scaler(sc_f, opt_f, max_grad_norm=1.0)  # one good step: state exists
    torch.cuda.synchronize()
    params_before = [p.detach().clone() for p in fused]
    steps_before = [float(opt_f.state[p]["step"]) for p in fused[:-1]]
    scale_before = sc_f.get_scale()
    _set_grads(fused, fused, gpu, 302, scale_before)

    def failing_launch(*args, **kwargs):
        raise _lib.HipKernelError("pt_adamw_step_scaled", _lib.PT_ELAUNCH, "forced by the test")

    monkeypatch.setattr(ops, "adamw_step_scaled", failing_launch)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # no fallback warning either
        with pytest.raises(FusedAdamWStepFailed):
            hook.step_with_grad_scaler(sc_f, opt_f, max_grad_norm=1.0)
    torch.cuda.synchronize()
    # the counters advanced once (by the fused path, before its launch failed), not twice
    assert [float(opt_f.state[p]["step"]) for p in fused[:-1]] == [s + 1 for s in steps_before]
    # no update was applied, by the fused kernel or by torch's step
    for p, before in zip(fused, params_before):
        assert torch.equal(p.detach(), before)


def test_a_failure_after_the_plain_step_began_is_not_retried(gpu, monkeypatch):
    from picotron_amd import _lib, ops
    from picotron_amd.nn.triton_kernels import FusedAdamWStepFailed

    fused, _, opt_f, _, _, _ = _setup(gpu, 400)
    _set_grads(fused, fused, gpu, 401, 1.0)
    hook = AdamWStepWithFallback(use_triton=True)
    hook.step(opt_f)
    torch.cuda.synchronize()
    params_before = [p.detach().clone() for p in fused]
    steps_before = [float(opt_f.state[p]["step"]) for p in fused[:-1]]

    def failing_launch(*args, **kwargs):
        raise _lib.HipKernelError("pt_adamw_step", _lib.PT_ELAUNCH, "forced by the test")

    monkeypatch.setattr(ops, "adamw_step", failing_launch)
    with pytest.raises(FusedAdamWStepFailed):
        hook.step(opt_f)
    assert [float(opt_f.state[p]["step"]) for p in fused[:-1]] == [s + 1 for s in steps_before]
    for p, before in zip(fused, params_before):
        assert torch.equal(p.detach(), before)
    # an optimizer the fused path rejects before changing anything still falls back
    sgd = torch.optim.SGD([fused[0]], lr=0.1)
    with pytest.warns(RuntimeWarning):
        AdamWStepWithFallback(use_triton=True).step(sgd)


@pytest.mark.parametrize("max_norm", [None, 1e-3, 1e4])
def test_capturable_optimizer_decides_the_overflow_on_the_device(gpu, max_norm):
    """A capturable optimizer whose state exists takes the path that reads nothing on the
    host: the guarded update skips itself on an overflow and only unscales, the step counts
    advance by 1 - found_inf.  It follows torch's sequence step for step as the host-read
    path does (a step that would create the state still reads the flag: the first one
    overflows here and may leave no state behind, the second creates it)."""

    fused, ref, _, opt_r, sc_f, sc_r = _setup(gpu, 15)
    opt_f = torch.optim.AdamW(fused, capturable=True, **HP)
    for step in range(8):
        scale = sc_r.get_scale()
        bad = OVERFLOWS.get(step)
        print(f"capturable grad scaler step {step} scale {scale} bad {bad} max_norm {max_norm}", flush=True)
        _set_grads(fused, ref, gpu, 100 * step, scale, bad)
        _reference_step(sc_r, opt_r, ref, max_norm)
        had_state = bool(opt_f.state)
        skipped = triton_grad_scaler_step(sc_f, opt_f, max_norm)
        if not had_state:
            # the step that would create the state reads the flag on the host (step 0
            # overflows and leaves none; step 1 creates it)
            assert skipped is (bad is not None)
            assert bool(opt_f.state) == (bad is None)
        else:
            assert isinstance(skipped, torch.Tensor) and bool(skipped.item()) == (bad is not None)
        _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too=bad is None or max_norm is None)
    assert sc_f.get_scale() == 2.0 ** 15


def test_captured_fp16_step_matches_eager_steps_through_overflows(gpu):
    """A whole fp16 training step -- the scaled loss's backward, then the fused unscale +
    clip + AdamW + scaler update -- captured in one HIP graph after warm-up and replayed over
    inputs of which some overflow (inf, then NaN): every replay leaves the parameters,
    moments, step counts, scale and growth tracker that the same steps leave when run
    eagerly with the same capturable optimizer."""

    sizes = [4097, 70_000]
    n_steps, warmup = 10, 3
    bad_steps = {4: float("inf"), 7: float("nan")}
    inputs = []
    for k in range(n_steps):
        x = [randn((n,), torch.float32, gpu, 900 + 10 * k + i, 1e-3) for i, n in enumerate(sizes)]
        if k in bad_steps:
            x[1][123] = bad_steps[k]
        inputs.append(x)

    def build():
        params = [torch.nn.Parameter(randn((n,), torch.float32, gpu, 40 + n, 0.02)) for n in sizes]
        opt = torch.optim.AdamW(params, capturable=True, **HP)
        sc = torch.amp.GradScaler("cuda", init_scale=2.0 ** 16, growth_interval=2)
        return params, opt, sc, AdamWStepWithFallback(use_triton=True)

    def step(run, x):
        params, opt, sc, stepper = run
        opt.zero_grad(set_to_none=False)
        loss = sum((p * xi).sum() for p, xi in zip(params, x))
        sc.scale(loss).backward()
        stepper.step_with_grad_scaler(sc, opt, 1.0)

    def state_of(run):
        params, opt, sc, _ = run
        out = [sc.get_scale(), int(sc._growth_tracker.item())]
        for p in params:
            st = opt.state[p]
            out.append((p.detach().clone(), st["exp_avg"].clone(), st["exp_avg_sq"].clone(), float(st["step"])))
        return out

    eager, graphed = build(), build()
    static_x = [t.clone() for t in inputs[0]]
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # no fallback
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for k in range(warmup):
                for s, t in zip(static_x, inputs[k]):
                    s.copy_(t)
                step(graphed, static_x)
        torch.cuda.current_stream().wait_stream(side)
        for k in range(warmup):
            step(eager, inputs[k])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(graphed, static_x)
        for k in range(warmup, n_steps):
            for s, t in zip(static_x, inputs[k]):
                s.copy_(t)
            graph.replay()
            step(eager, inputs[k])
            torch.cuda.synchronize()
            print(f"captured fp16 step {k} (bad {bad_steps.get(k)})", flush=True)
            a, b = state_of(graphed), state_of(eager)
            assert a[:2] == b[:2], f"step {k}: scale / growth tracker {a[:2]} against {b[:2]}"
            for (pa, ma, va, sa), (pb, mb, vb, sb) in zip(a[2:], b[2:]):
                assert sa == sb, f"step {k}: step count {sa} against {sb}"
                assert torch.equal(pa, pb) and torch.equal(ma, mb) and torch.equal(va, vb), f"step {k}"
    # two overflow steps were skipped: 10 steps, 8 applied
    assert state_of(eager)[2][3] == n_steps - len(bad_steps)


@pytest.mark.parametrize("both_capturable", [True, False])
def test_groups_decide_on_the_device_only_when_all_are_capturable(gpu, both_capturable):
    """Two parameter groups with their own learning rate and weight decay: with both
    capturable the overflow is decided on the device (a device flag is returned), with one
    not the host reads it; either way the steps follow torch's sequence through overflows."""

    fused, ref, _, _, sc_f, sc_r = _setup(gpu, 25)
    split = 4

    def groups(params, capturable):
        return [dict(params=params[:split], lr=3e-4, weight_decay=0.1, capturable=capturable[0]),
                dict(params=params[split:], lr=1e-3, weight_decay=0.0, capturable=capturable[1])]

    caps = (True, both_capturable)
    opt_f = torch.optim.AdamW(groups(fused, caps), betas=(0.9, 0.95), eps=1e-8)
    opt_r = torch.optim.AdamW(groups(ref, (False, False)), betas=(0.9, 0.95), eps=1e-8, foreach=False)
    for step in range(6):
        scale = sc_r.get_scale()
        bad = {2: float("inf"), 4: float("nan")}.get(step)
        print(f"groups step {step} scale {scale} bad {bad} capturable {caps}", flush=True)
        _set_grads(fused, ref, gpu, 700 + 100 * step, scale, bad)
        _reference_step(sc_r, opt_r, ref, 1.0)
        had_state = bool(opt_f.state)
        skipped = triton_grad_scaler_step(sc_f, opt_f, 1.0)
        if had_state and both_capturable:
            assert isinstance(skipped, torch.Tensor) and bool(skipped.item()) == (bad is not None)
        else:
            assert skipped is (bad is not None)
        _compare(fused, ref, opt_f, opt_r, sc_f, sc_r, grads_too=bad is None)
