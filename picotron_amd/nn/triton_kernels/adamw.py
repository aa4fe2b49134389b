"""Fused multi-tensor AdamW step on gfx950 behind picotron's Triton-AdamW hook.

Drop-in for ``picotron.nn.triton_kernels.adamw`` (reference
src/picotron/nn/triton_kernels/adamw.py), whose ``triton_adamw_step`` always raises and
whose ``AdamWStepWithFallback`` therefore always runs ``optimizer.step()``.  Here
``triton_adamw_step(optimizer)`` updates every parameter of a ``torch.optim.AdamW`` in one
HIP launch, keeping torch's state layout (``state[p] = {"step", "exp_avg", "exp_avg_sq"}``
with a CPU float32 ``step`` tensor) so ``optimizer.state_dict()`` / ``load_state_dict()``
and picotron's checkpoints (src/picotron/serialize/checkpoint.py:50,91) round-trip, and
falling back is always possible.  Hyperparameters are read from ``param_groups`` on every
call (the train loop rewrites ``lr`` each step, train_loop.py:127,328-335).

Supported: fp32 dense parameters and gradients on a gfx950 device, ``amsgrad=False``,
``maximize=False``, ``differentiable=False``, float ``lr``.  Anything else raises
:class:`TritonAdamWUnavailable` (a ``RuntimeError`` whose message says "not implemented"),
and the fallback runs torch's own step.  With ``capturable=True`` the step counts stay fp32
scalars on the device, advanced there, and the kernel reads them: no host value depends on
the step, so a whole training step (forward, backward, clipping, this update) can be
captured in a HIP graph and replayed.

``triton_clip_grad_norm_and_step(optimizer, max_norm)`` fuses the gradient clipping the
train loop runs right before the step (reference src/picotron/training/train_loop.py:163-168
and ``_clip_gradients`` :338-350, i.e. ``torch.nn.utils.clip_grad_norm_``): one kernel reads
the gradients for the norm and the clip coefficient stays on the device, where the step
applies it as it reads each gradient, instead of a separate read-modify-write pass.
"""

from __future__ import annotations

import threading
import warnings

import numpy as np
import torch
from torch import Tensor
from torch.optim import Optimizer

from picotron_amd import _lib, ops


class TritonAdamWUnavailable(RuntimeError):
    """Raised when the fused (HIP) AdamW step cannot run for this optimizer."""


class FusedAdamWStepFailed(RuntimeError):
    """The fused step failed after it had begun to change the optimizer's state or the
    gradients (step counters advanced, a gradient unscaled, an update launched).  Running
    torch's step after it would apply part of the update twice, so the fallbacks of
    :class:`AdamWStepWithFallback` let this error through instead of retrying."""


def _committed(fn, *args, **kwargs):
    """Runs the state-changing part of a fused step: any error becomes FusedAdamWStepFailed."""

    try:
        return fn(*args, **kwargs)
    except FusedAdamWStepFailed:
        raise
    except Exception as error:
        raise FusedAdamWStepFailed(
            f"the fused AdamW step failed after changing optimizer state: {error}") from error


def _reject(reason: str) -> TritonAdamWUnavailable:
    return TritonAdamWUnavailable(f"Fused HIP AdamW is not implemented for {reason}; using PyTorch AdamW instead.")


def _check_group(group: dict) -> None:
    for flag in ("amsgrad", "maximize", "differentiable"):
        if group.get(flag, False):
            raise _reject(f"{flag}=True")
    if group.get("fused"):
        raise _reject("fused=True optimizers")
    if not group.get("decoupled_weight_decay", True):
        raise _reject("Adam with coupled weight decay")
    for key in ("lr", "eps", "weight_decay"):
        if isinstance(group[key], Tensor):
            raise _reject(f"tensor-valued {key}")
    if any(isinstance(b, Tensor) for b in group["betas"]):
        raise _reject("tensor-valued betas")


def _check_param(p: Tensor, g: Tensor) -> None:
    if not p.is_cuda or not g.is_cuda:
        raise _reject("CPU tensors")
    if p.dtype != torch.float32 or g.dtype != torch.float32:
        raise _reject(f"{p.dtype} parameters")
    if g.is_sparse:
        raise _reject("sparse gradients")
    if not p.is_contiguous() or not g.is_contiguous() or g.device != p.device:
        raise _reject("non-contiguous parameters or gradients")


def _check_state(state: dict, p: Tensor, capturable: bool = False) -> None:
    """An existing optimizer state (resumed from a checkpoint, or written by torch's own step)
    must be what the kernel's raw pointers assume: fp32 contiguous moments of p's size on p's
    device and a one-element step tensor (for a capturable group an fp32 scalar on p's
    device).  ``Optimizer.load_state_dict`` does not check state shapes, and torch's step
    would raise on a mismatch where the kernel would read and write out of bounds."""

    if len(state) == 0:
        return
    step = state.get("step")
    if not isinstance(step, Tensor) or step.numel() != 1:
        raise _reject("optimizer states whose step is not a one-element tensor")
    if capturable and (step.device != p.device or step.dtype != torch.float32):
        raise _reject("capturable steps that are not fp32 scalars on the parameter's device")
    for key in ("exp_avg", "exp_avg_sq"):
        m = state.get(key)
        if not isinstance(m, Tensor):
            raise _reject(f"optimizer states without {key}")
        if m.dtype != torch.float32 or m.device != p.device or m.is_sparse:
            raise _reject(f"optimizer states whose {key} is not fp32 on the parameter's device")
        if m.numel() != p.numel() or not m.is_contiguous():
            raise _reject(f"optimizer states whose {key} does not match the parameter "
                          f"({tuple(m.shape)} for {tuple(p.shape)}, or not contiguous)")


_table_cache: dict[tuple, Tensor] = {}
_TABLE_CACHE_SIZE = 16
_table_lock = threading.Lock()  # optimizers may step from several threads at once
# Tables used while a stream is being captured into a graph: the graph's kernels read them
# on every replay, so they stay alive for the life of the process instead of leaving with
# the cache's eviction.
_captured_tables: list[Tensor] = []


def _device_table(host_table: Tensor, device: torch.device) -> Tensor:
    """The device copy of a record table, cached by content (tables repeat every step).

    Under graph capture the table must already be cached (by an eager call on the same
    tensors, as in the usual warm-up before a capture): building it there would need a
    pinned host allocation and a host-to-device copy inside the graph."""

    key = (device, host_table.numpy().tobytes())
    capturing = torch.cuda.is_current_stream_capturing()
    with _table_lock:
        cached = _table_cache.pop(key, None)
    if cached is None:
        if capturing:
            raise TritonAdamWUnavailable(
                "HIP AdamW: the tensor table is first built during graph capture; run the "
                "same call once before capturing it.")
        cached = host_table.pin_memory().to(device, non_blocking=True)
    with _table_lock:
        if capturing:
            _captured_tables.append(cached)
        _table_cache[key] = cached  # most recent last
        while len(_table_cache) > _TABLE_CACHE_SIZE:
            del _table_cache[next(iter(_table_cache))]
    return cached


def _plan(optimizer: Optimizer) -> tuple[list[tuple[dict, list[Tensor]]], torch.device | None]:
    """Validate everything the fused step needs, touching no state; returns the parameter
    groups with their parameters that have gradients, and the device."""

    if not isinstance(optimizer, torch.optim.AdamW):
        raise _reject(f"{type(optimizer).__name__} (only torch.optim.AdamW)")
    groups = []
    device = None
    state_of = optimizer.state
    for group in optimizer.param_groups:
        _check_group(group)
        capturable = bool(group.get("capturable", False))
        params = []
        for p in group["params"]:
            g = p.grad
            if g is None:
                continue
            state = state_of.get(p)
            if state:
                _check_state(state, p, capturable)
            _check_param(p, g)
            if device is None:
                device = p.device
            elif p.device != device:
                raise _reject("parameters on several devices")
            params.append(p)
        groups.append((group, params))
    if device is None:
        return groups, None
    reason = _lib.unavailable_reason()
    if reason is not None:
        raise TritonAdamWUnavailable(f"HIP kernel library unavailable: {reason}")
    if not ops.device_supported(device.index if device.index is not None else torch.cuda.current_device()):
        raise _reject("devices other than gfx950")
    # Every check that can fail happens before any optimizer state is touched, so a
    # fallback to optimizer.step() never sees a half-applied step.
    per_block = ops.adamw_block_elems()
    total = 0
    for _, params in groups:
        blocks = sum((p.numel() + per_block - 1) // per_block for p in params)
        total += blocks
        if blocks * 256 > 0xFFFFFFFF:
            raise _reject("parameter groups above 2^24 blocks of elements")
    if total * 256 > 0xFFFFFFFF:
        raise _reject("more than 2^24 blocks of gradient elements")
    return groups, device


def _prepare(optimizer: Optimizer, groups, device: torch.device) -> tuple[list, list[Tensor]]:
    """Host side of the fused step, touching no step counter: lazy state creation as
    torch.optim.Adam._init_group does for the non-fused case (a CPU fp32 step, or for a
    capturable group an fp32 step on the parameter's device; zeroed moments of the
    parameter's shape, here views of one allocation per group), and the record tables: one per
    distinct next step value, or for a capturable group one with the table of its device
    steps.  Returns the launches and the parameters whose state was created here (so that a
    skipped step can remove it again)."""

    launches = []
    created = []
    state_of = optimizer.state
    for group, params in groups:
        if not params:
            continue
        beta1, beta2 = group["betas"]
        capturable = bool(group.get("capturable", False))
        fresh = [p for p in params if len(state_of[p]) == 0]
        # the group's new moments come from one allocation (ops.adamw_moments)
        moments = iter(ops.adamw_moments(fresh))
        states = []
        for p in params:
            state = state_of[p]
            if len(state) == 0:
                if capturable:
                    state["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
                else:
                    state["step"] = torch.tensor(0.0, dtype=torch.float32)
                state["exp_avg"], state["exp_avg_sq"] = next(moments)
                created.append(p)
            states.append(state)
        hyper = dict(lr=group["lr"], beta1=beta1, beta2=beta2, eps=group["eps"],
                     weight_decay=group["weight_decay"])
        if capturable:
            # the step values stay on the device: no host read, one launch for the group
            buckets = [(None, params, states)]
        else:
            # one launch per distinct step count (usually one for the whole group); the value
            # is the one `state["step"] += 1` leaves in the float32 tensor
            values = [state["step"].item() for state in states]
            if values.count(values[0]) == len(values):
                buckets = [(_next_step(values[0]), params, states)]
            else:
                by_step: dict[float, tuple[list, list]] = {}
                for p, state, value in zip(params, states, values):
                    ps, sts = by_step.setdefault(_next_step(value), ([], []))
                    ps.append(p)
                    sts.append(state)
                buckets = [(step, ps, sts) for step, (ps, sts) in by_step.items()]
        for step, ps, sts in buckets:
            host_table, total_blocks = ops.adamw_table(
                ps, [p.grad for p in ps], [st["exp_avg"] for st in sts],
                [st["exp_avg_sq"] for st in sts])
            if total_blocks == 0:
                continue
            table = _device_table(host_table, device)
            if step is None:
                steps = _device_table(ops.adamw_step_table(ps, [st["step"] for st in sts]), device)
                launches.append((table, total_blocks, steps, hyper))
            else:
                launches.append((table, total_blocks, None, dict(hyper, step=step)))
    return launches, created


def _next_step(value: float) -> float:
    return float(np.float32(value) + np.float32(1.0))


def _launch(optimizer: Optimizer, groups, launches: list, grad_scale: Tensor | None,
            write_grad: bool) -> None:
    """Advances every stepped parameter's step counter (as torch's AdamW does: on the host,
    or for a capturable group on the device) and launches the prepared updates.  It changes
    state from its first line, so any error in it is FusedAdamWStepFailed."""

    _committed(_launch_all, optimizer, groups, launches, grad_scale, write_grad)


def _launch_all(optimizer: Optimizer, groups, launches: list, grad_scale: Tensor | None,
                write_grad: bool) -> None:
    state_of = optimizer.state
    for group, params in groups:
        if params:
            # float32 step tensors on the host, or on the device for a capturable group: one
            # call adds 1 to all of them, the same float32 addition as `step += 1` on each
            torch._foreach_add_([state_of[p]["step"] for p in params], 1.0)
    for table, total_blocks, steps, hyper in launches:
        if steps is not None:
            ops.adamw_step_device_step(table, total_blocks, steps, grad_scale=grad_scale,
                                       write_grad=write_grad, **hyper)
        elif grad_scale is None:
            ops.adamw_step(table, total_blocks, **hyper)
        else:
            ops.adamw_step_scaled(table, total_blocks, grad_scale, write_grad=write_grad, **hyper)


def _run(optimizer: Optimizer, groups, device: torch.device, grad_scale: Tensor | None,
         write_grad: bool) -> None:
    launches, _ = _prepare(optimizer, groups, device)
    _launch(optimizer, groups, launches, grad_scale, write_grad)


def triton_adamw_step(optimizer: Optimizer) -> None:
    """One AdamW step of ``optimizer`` with the fused HIP kernel (or raise unavailable)."""

    groups, device = _plan(optimizer)
    if device is not None:
        _run(optimizer, groups, device, None, False)


def triton_clip_grad_norm_and_step(
    optimizer: Optimizer, max_norm: float, *, write_back_grads: bool = True
) -> Tensor:
    """``torch.nn.utils.clip_grad_norm_(params, max_norm)`` followed by ``optimizer.step()``
    for a ``torch.optim.AdamW``, fused: returns the total gradient norm (fp32 scalar tensor).

    The norm covers every parameter of the optimizer that has a gradient (the train loop's
    model.parameters()).  With ``write_back_grads`` the gradients are left clipped, exactly
    as ``clip_grad_norm_`` leaves them; without it they keep their unclipped values (one
    write of every gradient less) while the update still uses the clipped ones.
    """

    groups, device = _plan(optimizer)
    if device is None:
        return torch.tensor(0.0)
    grads = [p.grad for _, params in groups for p in params]
    host_table, total_blocks = ops.adamw_table(grads, grads, grads, grads)
    total_norm, coef = ops.clip_grad_norm(_device_table(host_table, device), total_blocks, float(max_norm))
    _run(optimizer, groups, device, coef, write_back_grads)
    return total_norm


# ------------------------------------------------------------------ loss scaling and ZeRO
#
# The mixed-precision / ZeRO path of the reference (src/picotron/parallel/zero.py) handles
# gradients outside the optimizer: DistributedGradScaler.step (:50-79) calls
# ZeroOptimizer.unscale_and_check_ (:139-163; a finite check per parameter, each a host
# sync, then g *= 1/scale), ZeroOptimizer.clip_grad_norm_ (:165-186; g *= coef when coef < 1)
# and the inner torch AdamW step (:130-137).  The functions below run that on one rank
# with one read of the gradients for all statistics and a single host sync.


def _grads_of(parameters) -> tuple[list[Tensor], torch.device | None]:
    grads = [p.grad for p in parameters if p.grad is not None]
    device = None
    for g in grads:
        if not g.is_cuda or g.dtype != torch.float32 or g.is_sparse or not g.is_contiguous():
            raise _reject("gradients that are not dense contiguous fp32 GPU tensors")
        if device is None:
            device = g.device
        elif g.device != device:
            raise _reject("gradients on several devices")
    if device is not None:
        reason = _lib.unavailable_reason()
        if reason is not None:
            raise TritonAdamWUnavailable(f"HIP kernel library unavailable: {reason}")
        if not ops.device_supported(device.index if device.index is not None else torch.cuda.current_device()):
            raise _reject("devices other than gfx950")
    return grads, device


def _grad_table(grads: list[Tensor], device: torch.device) -> tuple[Tensor, int]:
    host_table, blocks = ops.adamw_table(grads, grads, grads, grads)
    if blocks * 256 > 0xFFFFFFFF:
        raise _reject("more than 2^24 blocks of gradient elements")
    return _device_table(host_table, device), blocks


def triton_unscale_and_check_(parameters, scale: float) -> bool:
    """``ZeroOptimizer.unscale_and_check_`` on one rank: True (gradients untouched) if any
    gradient is inf or NaN, else every gradient is multiplied by ``1 / scale`` and False."""

    if scale <= 0:
        raise ValueError("loss scale must be positive.")
    grads, device = _grads_of(parameters)
    if device is None:
        return False
    table, blocks = _grad_table(grads, device)
    inv = torch.full((), 1.0 / scale, dtype=torch.float32, device=device)
    _, multiplier, found_inf = ops.grad_stats(table, blocks, inv)
    if bool(found_inf.item()):
        return True
    ops.grad_scale(table, blocks, multiplier)
    return False


def triton_zero_clip_grad_norm_(parameters, max_norm: float) -> Tensor:
    """``ZeroOptimizer.clip_grad_norm_`` on one rank: returns the total norm and multiplies
    every gradient by ``max_norm / (total_norm + 1e-6)`` when that is below 1, without a
    host sync (the comparison happens on the device)."""

    if max_norm <= 0:
        raise ValueError("max_norm must be positive.")
    grads, device = _grads_of(parameters)
    if device is None:
        return torch.tensor(0.0)
    table, blocks = _grad_table(grads, device)
    total, multiplier, _ = ops.grad_stats(table, blocks, None, max_norm, ops.CLIP_IF_BELOW_ONE)
    ops.grad_scale(table, blocks, multiplier)
    return total


def triton_unscale_clip_and_step(
    optimizer: Optimizer, scale: float, max_norm: float | None = None, *, parameters=None
) -> bool:
    """The ZeRO mixed-precision update on one rank, fused: ``unscale_and_check_(scale)``,
    then (if every gradient is finite) ``clip_grad_norm_(max_norm)`` and the AdamW step of
    ``optimizer`` (the ZeRO optimizer's inner ``torch.optim.AdamW``).

    One pass reads every gradient of ``parameters`` (default: the optimizer's) for the
    finite check, the norm of the unscaled gradients and the combined unscale x clip
    multiplier; one host sync reads the finite flag; the step then applies the multiplier
    as it reads each gradient and writes the unscaled, clipped gradient back.  Gradients of
    ``parameters`` outside the optimizer are rescaled in place as the reference does.
    Returns True (nothing changed) when a gradient is inf or NaN, like
    ``unscale_and_check_``.
    """

    if scale <= 0:
        raise ValueError("loss scale must be positive.")
    if max_norm is not None and max_norm <= 0:
        raise ValueError("max_norm must be positive.")
    groups, device = _plan(optimizer)
    owned = [p for _, params in groups for p in params]
    if parameters is None:
        parameters = owned
    grads, gdevice = _grads_of(parameters)
    if gdevice is None:
        return False
    if device is not None and device != gdevice:
        raise _reject("gradients on several devices")
    table, blocks = _grad_table(grads, gdevice)
    # a fill kernel, not a host-to-device copy (which would wait for the stream)
    inv = torch.full((), 1.0 / scale, dtype=torch.float32, device=gdevice)
    _, multiplier, found_inf = ops.grad_stats(table, blocks, inv, max_norm, ops.CLIP_IF_BELOW_ONE)
    # All host work of the update happens before the flag is read, so that the device idles
    # only for the launches after it.
    owned_ids = {id(p) for p in owned}
    others = [p.grad for p in parameters if p.grad is not None and id(p) not in owned_ids]
    other = _grad_table(others, gdevice) if others else None
    launches, created = _prepare(optimizer, groups, device) if device is not None else ([], [])
    if bool(found_inf.item()):
        for p in created:  # a skipped step leaves no state behind, as in the reference
            del optimizer.state[p]
        return True
    if other is not None:
        ops.grad_scale(other[0], other[1], multiplier)
    if device is not None:
        _launch(optimizer, groups, launches, multiplier, True)
    return False


def triton_grad_scaler_step(grad_scaler, optimizer: Optimizer,
                            max_norm: float | None = None) -> bool | Tensor:
    """The train loop's single-GPU fp16 update, fused: ``grad_scaler.unscale_(optimizer)``,
    ``torch.nn.utils.clip_grad_norm_(params, max_norm)`` (when ``max_norm`` is given),
    ``grad_scaler.step(optimizer)`` and ``grad_scaler.update()`` (reference
    src/picotron/training/train_loop.py:155-160, with the ``torch.amp.GradScaler`` created at
    :285-296 for fp16 without ZeRO and ``_clip_gradients`` at :338-350).

    One pass reads every gradient for the finite check, the norm of the unscaled gradients and
    the combined multiplier ``inv_scale * clip_coef`` (``inv_scale`` is the scaler's
    ``1 / scale`` computed as ``unscale_`` computes it, in double then rounded to fp32); one
    host read of the finite flag, as ``grad_scaler.step`` makes; then the AdamW step applies the
    multiplier as it reads each gradient and writes the unscaled, clipped gradient back.  When a
    gradient is inf or NaN the step is skipped (no state is created or advanced), the gradients
    are left unscaled as ``unscale_`` leaves them (with ``max_norm``, torch's
    ``clip_grad_norm_`` would then also multiply them by a coefficient computed from the
    non-finite norm, zero or NaN; here they are not clipped, and the next ``zero_grad`` discards
    them either way), and the scaler backs off exactly as torch's:
    the flag is recorded in the scaler's per-optimizer state as ``unscale_`` records it, and
    ``grad_scaler.update()`` consumes it.  Returns True when the step was skipped.

    For an optimizer whose groups are all ``capturable=True`` and whose state exists (every
    step after the first), nothing is read on the host: the AdamW launch reads the flag on
    the device and either updates or only unscales, and the step counts advance by
    ``1 - found_inf`` -- the same results, in a form a HIP graph can capture (warm up before
    capturing; a step that would create state reads the flag as above).  The return value is
    then the flag itself, a one-element int32 device tensor (nonzero when skipped).

    With a power-of-two scale (torch's defaults: 65536, growth 2, backoff 0.5) the unscaled
    gradients are bitwise torch's; the clip coefficient follows torch's formula with the norm
    summed in a different order (fp32 rounding of the last bits).
    """

    from torch.amp.grad_scaler import OptState

    if not isinstance(grad_scaler, torch.amp.GradScaler):
        raise _reject(f"{type(grad_scaler).__name__} (only torch.amp.GradScaler)")
    if max_norm is not None and max_norm <= 0:
        raise ValueError("max_norm must be positive.")
    if not grad_scaler.is_enabled():
        if max_norm is None:
            triton_adamw_step(optimizer)
        else:
            triton_clip_grad_norm_and_step(optimizer, max_norm)
        return False
    scale, _ = grad_scaler._check_scale_growth_tracker("step")
    state = grad_scaler._per_optimizer_states[id(optimizer)]
    if state["stage"] is not OptState.READY:
        raise _reject("a GradScaler that already unscaled or stepped this optimizer this iteration")
    groups, device = _plan(optimizer)
    if device is None:
        raise _reject("an optimizer without gradients")
    if scale.device != device:
        raise _reject("a loss scale on another device than the gradients")
    grads = [p.grad for _, params in groups for p in params]
    table, blocks = _grad_table(grads, device)
    # every check that can fail is done: from here on the call runs to the end, and an error
    # (a failed launch) is FusedAdamWStepFailed, never a reason to run torch's sequence again
    return _committed(_grad_scaler_step_committed, grad_scaler, state, optimizer, groups,
                      device, scale, table, blocks, max_norm)


def _grad_scaler_step_committed(grad_scaler, state, optimizer, groups, device, scale, table,
                                blocks, max_norm) -> bool | Tensor:
    from torch.amp.grad_scaler import OptState

    inv_scale = scale.double().reciprocal().float()
    _, multiplier, found_inf = ops.grad_stats(
        table, blocks, inv_scale, max_norm, ops.CLIP_CLAMP)
    launches, created = _prepare(optimizer, groups, device)
    if launches and not created and all(steps is not None for _, _, steps, _ in launches):
        # Every group capturable and its state in place: the overflow is decided on the
        # device -- the guarded update skips itself and only unscales, the step counts
        # advance by 1 - found_inf -- with no host read, so the update can be captured.
        keep = (1.0 - found_inf.float()).reshape(())
        steps_of = [optimizer.state[p]["step"] for _, params in groups for p in params]
        # the list overload adds on the device (the 0-dim tensor overload reads the value
        # on the host); step + 1.0 is the float32 addition of `step += 1`, step + 0.0 none
        torch._foreach_add_(steps_of, [keep] * len(steps_of))
        for launch_table, total_blocks, steps, hyper in launches:
            ops.adamw_step_device_step(launch_table, total_blocks, steps, grad_scale=multiplier,
                                       write_grad=True, found_inf=found_inf,
                                       inv_scale=inv_scale.reshape(1), **hyper)
        skipped = found_inf
    else:
        skipped = bool(found_inf.item())
        if skipped:
            for p in created:  # a skipped step leaves no state behind
                del optimizer.state[p]
            ops.grad_scale(table, blocks, inv_scale)
        else:
            _launch(optimizer, groups, launches, multiplier, True)
    state["found_inf_per_device"] = {device: found_inf.float()}
    state["stage"] = OptState.STEPPED
    grad_scaler.update()
    return skipped


class AdamWStepWithFallback:
    """Attempt the fused step when enabled, else (or on failure) ``optimizer.step()``
    (reference adamw.py:27-47)."""

    def __init__(self, *, use_triton: bool = False) -> None:
        self.use_triton = use_triton
        self._fallback_warned = False

    def step(self, optimizer: Optimizer, max_grad_norm: float | None = None) -> None:
        """``optimizer.step()``; with ``max_grad_norm`` the gradients are first clipped as
        ``torch.nn.utils.clip_grad_norm_`` does (fused into the step on the fast path).  An
        error raised after the fused step began to change state (FusedAdamWStepFailed)
        propagates: torch's step is run only when nothing has been changed yet."""

        if self.use_triton:
            try:
                if max_grad_norm is None:
                    triton_adamw_step(optimizer)
                else:
                    triton_clip_grad_norm_and_step(optimizer, max_grad_norm)
                return
            except FusedAdamWStepFailed:
                raise
            except Exception as error:
                if not self._fallback_warned:
                    warnings.warn(
                        f"Triton AdamW unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._fallback_warned = True
        if max_grad_norm is not None:
            params = [p for group in optimizer.param_groups for p in group["params"]]
            torch.nn.utils.clip_grad_norm_(params, max_grad_norm)
        optimizer.step()

    def step_with_grad_scaler(self, grad_scaler, optimizer: Optimizer,
                              max_grad_norm: float | None = None) -> None:
        """The train loop's fp16 update (reference src/picotron/training/train_loop.py:155-160):
        ``grad_scaler.unscale_``, ``clip_grad_norm_`` when ``max_grad_norm`` is given,
        ``grad_scaler.step`` and ``grad_scaler.update``; fused on the fast path
        (:func:`triton_grad_scaler_step`), else exactly that torch sequence (not after an
        error raised once the fused update began: FusedAdamWStepFailed propagates)."""

        if self.use_triton:
            try:
                triton_grad_scaler_step(grad_scaler, optimizer, max_grad_norm)
                return
            except FusedAdamWStepFailed:
                raise
            except Exception as error:
                if not self._fallback_warned:
                    warnings.warn(
                        f"Triton AdamW unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._fallback_warned = True
        grad_scaler.unscale_(optimizer)
        if max_grad_norm is not None:
            params = [p for group in optimizer.param_groups for p in group["params"]]
            torch.nn.utils.clip_grad_norm_(params, max_grad_norm)
        grad_scaler.step(optimizer)
        grad_scaler.update()
