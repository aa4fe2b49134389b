"""Fused RMSNorm forward and backward on gfx950 behind picotron's Triton-RMSNorm surface.

Drop-in for ``picotron.nn.triton_kernels.rmsnorm`` (reference
src/picotron/nn/triton_kernels/rmsnorm.py): same public names, autograd Function
signature ``apply(hidden_states, weight, eps, use_fast_forward)``, exception type and
validation behaviour.  The reference runs a Triton forward plus a separate PyTorch
``_inverse_rms`` pass and an eager PyTorch backward; here both directions are HIP kernels
(``pt_rmsnorm_fwd`` writes y and the fp32 rstd in one pass, ``pt_rmsnorm_bwd`` writes dx
and a deterministic dW).  The PyTorch path (``use_fast_forward=False``) is the
reference's own CPU-verifiable formula.

``triton_residual_rms_norm(x, residual, weight, eps)`` fuses the decoder block's residual
add with the norm that follows it (reference src/picotron/models/picotron_decoder.py:116-119:
``hidden = hidden + attention(...)`` then ``mlp_norm(hidden)``): it returns ``(h, y)`` with
``h = x + residual`` and ``y = RMSNorm(h)`` from one pass, and its backward adds the
gradient arriving at ``h`` from the block's final residual add into the norm's input
gradient in the same pass.
"""

from __future__ import annotations

import warnings

import torch
from torch import Tensor

from picotron_amd import _lib, ops
from picotron_amd.nn.triton_kernels._gate import require_hip


class TritonRMSNormUnavailable(RuntimeError):
    """Raised when the fused (HIP) RMSNorm path cannot safely run."""


def _inverse_rms(hidden_states: Tensor, eps: float) -> Tensor:
    """Per-row inverse RMS in fp32, shape ``[..., 1]`` (reference rmsnorm.py:49-53)."""

    values = hidden_states.float()
    return torch.rsqrt(values.square().mean(dim=-1, keepdim=True) + eps)


def _pytorch_forward(hidden_states: Tensor, weight: Tensor, inverse_rms: Tensor) -> Tensor:
    """fp32 forward stored in the input dtype (reference rmsnorm.py:56-60)."""

    output = hidden_states.float() * inverse_rms * weight.float()
    return output.to(dtype=hidden_states.dtype)


def _pytorch_backward(
    hidden_states: Tensor, weight: Tensor, inverse_rms: Tensor, grad_output: Tensor
) -> tuple[Tensor, Tensor]:
    """Eager fp32 backward (reference rmsnorm.py:110-134)."""

    x = hidden_states.float()
    w = weight.float()
    g = grad_output.float()
    weighted_grad = g * w
    dot_mean = (weighted_grad * x).mean(dim=-1, keepdim=True)
    grad_x = inverse_rms * (weighted_grad - x * inverse_rms.square() * dot_mean)
    grad_w = (g * x * inverse_rms).reshape(-1, weight.numel()).sum(dim=0)
    return grad_x.to(dtype=hidden_states.dtype), grad_w.to(dtype=weight.dtype)


_backward_fallback_warned = False


def _kernel_backward() -> bool:
    """Whether a backward runs the HIP kernel.  A backward that builds a graph itself
    (``create_graph=True``, for higher-order gradients) takes the reference's eager formula
    instead (rmsnorm.py:110-134), which autograd can differentiate again as in the reference;
    the kernel's gradient would enter that graph as a constant."""

    return not torch.is_grad_enabled() or ops._compiling()


def _warn_backward_fallback(error: Exception) -> None:
    global _backward_fallback_warned
    if not _backward_fallback_warned:
        warnings.warn(
            f"HIP RMSNorm backward unavailable; using PyTorch fallback: {error}",
            RuntimeWarning,
            stacklevel=3,
        )
        _backward_fallback_warned = True


class _RMSNormAutogradFunction(torch.autograd.Function):
    """RMSNorm with a fused HIP forward and backward (or the PyTorch reference path)."""

    @staticmethod
    def forward(
        ctx: torch.autograd.function.FunctionCtx,
        hidden_states: Tensor,
        weight: Tensor,
        eps: float,
        use_triton_forward: bool,
    ) -> Tensor:
        ctx.use_hip = bool(use_triton_forward)
        if ctx.use_hip:
            output, rstd = ops.rmsnorm_fwd(hidden_states, weight, eps)
            ctx.save_for_backward(hidden_states, weight, rstd)
            return output
        inverse_rms = _inverse_rms(hidden_states, eps)
        ctx.save_for_backward(hidden_states, weight, inverse_rms)
        return _pytorch_forward(hidden_states, weight, inverse_rms)

    @staticmethod
    def backward(
        ctx: torch.autograd.function.FunctionCtx, grad_output: Tensor
    ) -> tuple[Tensor | None, Tensor | None, None, None]:
        hidden_states, weight, saved_rms = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if ctx.use_hip:
            if _kernel_backward():
                try:
                    grad_x, grad_w = ops.rmsnorm_bwd(
                        grad_output, hidden_states, weight, saved_rms, need_dx=need_x, need_dw=need_w
                    )
                    return grad_x, grad_w, None, None
                except _lib.HipKernelError as error:
                    # The reference backward cannot fail (it is eager PyTorch); keep that
                    # guarantee by recomputing with its formula.
                    _warn_backward_fallback(error)
            saved_rms = saved_rms.unsqueeze(-1)
        grad_x, grad_w = _pytorch_backward(hidden_states, weight, saved_rms, grad_output)
        return (grad_x if need_x else None), (grad_w if need_w else None), None, None


def _validate_triton_inputs(hidden_states: Tensor, weight: Tensor) -> None:
    """Launch constraints of the fused path (reference rmsnorm.py:137-149)."""

    require_hip(TritonRMSNormUnavailable, "RMSNorm", hidden_states, weight)
    if hidden_states.ndim < 1 or hidden_states.size(-1) != weight.numel():
        raise TritonRMSNormUnavailable("RMSNorm hidden size must match the weight size.")
    if weight.ndim != 1:
        raise TritonRMSNormUnavailable("RMSNorm weight must be 1-D.")
    if hidden_states.dtype not in (torch.float32, torch.float16, torch.bfloat16) or (
        weight.dtype not in (torch.float32, torch.float16, torch.bfloat16)
    ):
        raise TritonRMSNormUnavailable("HIP RMSNorm supports float32, float16 and bfloat16.")
    if not hidden_states.is_contiguous() or not weight.is_contiguous():
        raise TritonRMSNormUnavailable("HIP RMSNorm requires contiguous inputs.")


def triton_rms_norm(hidden_states: Tensor, weight: Tensor, eps: float) -> Tensor:
    """Fused RMSNorm (HIP forward and backward).

    Callers should catch :class:`TritonRMSNormUnavailable` and use their native RMSNorm
    when the GPU requirements are unmet (reference rmsnorm.py:152-160).
    """

    _validate_triton_inputs(hidden_states, weight)
    return _RMSNormAutogradFunction.apply(hidden_states, weight, eps, True)


def rms_norm_with_pytorch_forward(hidden_states: Tensor, weight: Tensor, eps: float) -> Tensor:
    """The reference's CPU-verifiable entry point: PyTorch forward and backward through the
    same autograd Function (reference rmsnorm.py:163-171)."""

    return _RMSNormAutogradFunction.apply(hidden_states, weight, eps, False)


class _ResidualRMSNormFunction(torch.autograd.Function):
    """(h, y) = (x + residual, RMSNorm(x + residual)) with fused HIP forward and backward."""

    @staticmethod
    def forward(ctx, x: Tensor, residual: Tensor, weight: Tensor, eps: float):  # type: ignore[override]
        h, y, rstd = ops.residual_rmsnorm_fwd(x, residual, weight, eps)
        ctx.save_for_backward(h, weight, rstd)
        ctx.set_materialize_grads(False)
        return h, y

    @staticmethod
    def backward(ctx, grad_h: Tensor | None, grad_y: Tensor | None):  # type: ignore[override]
        h, weight, rstd = ctx.saved_tensors
        need_x, need_r, need_w = ctx.needs_input_grad[:3]
        grad_w = None
        if grad_y is None:
            grad = grad_h
        else:
            grad = None
            if _kernel_backward():
                try:
                    grad, grad_w = ops.residual_rmsnorm_bwd(grad_y, grad_h, h, weight, rstd, need_dw=need_w)
                except _lib.HipKernelError as error:
                    _warn_backward_fallback(error)
            if grad is None:
                grad, grad_w = _pytorch_backward(h, weight, rstd.unsqueeze(-1), grad_y)
                if grad_h is not None:
                    grad = (grad.float() + grad_h.float()).to(h.dtype)
        return (grad if need_x else None), (grad if need_r else None), (grad_w if need_w else None), None


def triton_residual_rms_norm(
    hidden_states: Tensor, residual: Tensor, weight: Tensor, eps: float
) -> tuple[Tensor, Tensor]:
    """``h = hidden_states + residual`` and ``RMSNorm(h)`` fused; returns ``(h, y)``.

    Raises :class:`TritonRMSNormUnavailable` when the fused path cannot run (callers then
    add and normalise with PyTorch).
    """

    _validate_triton_inputs(hidden_states, weight)
    require_hip(TritonRMSNormUnavailable, "RMSNorm", residual)
    if residual.shape != hidden_states.shape or residual.dtype != hidden_states.dtype:
        raise TritonRMSNormUnavailable("residual must match hidden_states in shape and dtype.")
    if not residual.is_contiguous():
        raise TritonRMSNormUnavailable("HIP RMSNorm requires contiguous inputs.")
    return _ResidualRMSNormFunction.apply(hidden_states, residual, weight, eps)
