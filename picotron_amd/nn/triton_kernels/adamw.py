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
``maximize=False``, ``capturable=False``, ``differentiable=False``, float ``lr``.  Anything
else raises :class:`TritonAdamWUnavailable` (a ``RuntimeError`` whose message says "not
implemented"), and the fallback runs torch's own step.
"""

from __future__ import annotations

import warnings

import torch
from torch import Tensor
from torch.optim import Optimizer

from picotron_amd import _lib, ops


class TritonAdamWUnavailable(RuntimeError):
    """Raised when the fused (HIP) AdamW step cannot run for this optimizer."""


def _reject(reason: str) -> TritonAdamWUnavailable:
    return TritonAdamWUnavailable(f"Fused HIP AdamW is not implemented for {reason}; using PyTorch AdamW instead.")


def _check_group(group: dict) -> None:
    for flag in ("amsgrad", "maximize", "capturable", "differentiable"):
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


def _check_param(p: Tensor) -> None:
    if not p.is_cuda or not p.grad.is_cuda:
        raise _reject("CPU tensors")
    if p.dtype != torch.float32 or p.grad.dtype != torch.float32:
        raise _reject(f"{p.dtype} parameters")
    if p.grad.is_sparse:
        raise _reject("sparse gradients")
    if not p.is_contiguous() or not p.grad.is_contiguous() or p.grad.device != p.device:
        raise _reject("non-contiguous parameters or gradients")


_table_cache: dict[tuple, Tensor] = {}


def _device_table(key: tuple, host_table: Tensor, device: torch.device) -> Tensor:
    cached = _table_cache.get(key)
    if cached is not None:
        return cached
    _table_cache.clear()
    table = host_table.pin_memory().to(device, non_blocking=True)
    _table_cache[key] = table
    return table


def triton_adamw_step(optimizer: Optimizer) -> None:
    """One AdamW step of ``optimizer`` with the fused HIP kernel (or raise unavailable)."""

    if not isinstance(optimizer, torch.optim.AdamW):
        raise _reject(f"{type(optimizer).__name__} (only torch.optim.AdamW)")
    groups = []
    device = None
    for group in optimizer.param_groups:
        _check_group(group)
        params = [p for p in group["params"] if p.grad is not None]
        for p in params:
            _check_param(p)
            if device is None:
                device = p.device
            elif p.device != device:
                raise _reject("parameters on several devices")
        groups.append((group, params))
    if device is None:
        return
    reason = _lib.unavailable_reason()
    if reason is not None:
        raise TritonAdamWUnavailable(f"HIP kernel library unavailable: {reason}")
    if not ops.device_supported(device.index if device.index is not None else torch.cuda.current_device()):
        raise _reject("devices other than gfx950")
    # Every check that can fail happens before any optimizer state is touched, so a
    # fallback to optimizer.step() never sees a half-applied step.
    per_block = ops.adamw_block_elems()
    for _, params in groups:
        blocks = sum((p.numel() + per_block - 1) // per_block for p in params)
        if blocks * 256 > 0xFFFFFFFF:
            raise _reject("parameter groups above 2^24 blocks of elements")

    for group, params in groups:
        if not params:
            continue
        beta1, beta2 = group["betas"]
        # Lazy state creation and step increment exactly as torch.optim.Adam._init_group /
        # _single_tensor_adam do for the non-capturable, non-fused case.
        by_step: dict[float, list[Tensor]] = {}
        for p in params:
            state = optimizer.state[p]
            if len(state) == 0:
                state["step"] = torch.tensor(0.0, dtype=torch.float32)
                state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
            state["step"] += 1
            by_step.setdefault(float(state["step"].item()), []).append(p)
        for step, ps in by_step.items():
            grads = [p.grad for p in ps]
            exp_avgs = [optimizer.state[p]["exp_avg"] for p in ps]
            exp_avg_sqs = [optimizer.state[p]["exp_avg_sq"] for p in ps]
            host_table, total_blocks = ops.adamw_table(ps, grads, exp_avgs, exp_avg_sqs)
            if total_blocks == 0:
                continue
            key = tuple(host_table.flatten().tolist())
            table = _device_table(key, host_table, device)
            ops.adamw_step(
                table, total_blocks, lr=group["lr"], beta1=beta1, beta2=beta2, eps=group["eps"],
                weight_decay=group["weight_decay"], step=step,
            )


class AdamWStepWithFallback:
    """Attempt the fused step when enabled, else (or on failure) ``optimizer.step()``
    (reference adamw.py:27-47)."""

    def __init__(self, *, use_triton: bool = False) -> None:
        self.use_triton = use_triton
        self._fallback_warned = False

    def step(self, optimizer: Optimizer) -> None:
        if self.use_triton:
            try:
                triton_adamw_step(optimizer)
                return
            except Exception as error:
                if not self._fallback_warned:
                    warnings.warn(
                        f"Triton AdamW unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._fallback_warned = True
        optimizer.step()
