"""Fused SwiGLU activation forward and backward on gfx950 behind picotron's Triton-SwiGLU
surface.

Drop-in for ``picotron.nn.triton_kernels.swiglu`` (reference
src/picotron/nn/triton_kernels/swiglu.py): same public names, autograd Function signature
``apply(gate, up, use_fast_forward)``, exception type and validation.  The reference has a
Triton forward and an eager backward in the input dtype; here both are one-pass HIP
kernels computing in fp32 (``pt_swiglu_fwd`` / ``pt_swiglu_bwd``).
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.nn import functional as F

from picotron_amd import ops
from picotron_amd.nn.triton_kernels._gate import require_hip


class TritonSwiGLUUnavailable(RuntimeError):
    """Raised when the fused (HIP) SwiGLU path cannot safely run."""


class _SwiGLUAutogradFunction(torch.autograd.Function):
    """silu(gate) * up with a fused HIP forward/backward (or the PyTorch reference path)."""

    @staticmethod
    def forward(
        ctx: torch.autograd.function.FunctionCtx,
        gate: Tensor,
        up: Tensor,
        use_triton_forward: bool,
    ) -> Tensor:
        ctx.save_for_backward(gate, up)
        ctx.use_hip = bool(use_triton_forward)
        if ctx.use_hip:
            return ops.swiglu_fwd(gate, up)
        return F.silu(gate) * up

    @staticmethod
    def backward(
        ctx: torch.autograd.function.FunctionCtx, grad_output: Tensor
    ) -> tuple[Tensor | None, Tensor | None, None]:
        gate, up = ctx.saved_tensors
        # A backward that builds a graph itself (create_graph=True) takes the reference's
        # eager formula below, which autograd can differentiate again.
        if ctx.use_hip and (not torch.is_grad_enabled() or ops._compiling()):
            grad_gate, grad_up = ops.swiglu_bwd(
                grad_output, gate, up, ctx.needs_input_grad[0], ctx.needs_input_grad[1]
            )
            return grad_gate, grad_up, None
        # Reference backward (swiglu.py:71-81), in the input dtype.
        sigmoid_gate = torch.sigmoid(gate)
        silu_gate = gate * sigmoid_gate
        silu_derivative = sigmoid_gate * (1 + gate * (1 - sigmoid_gate))
        grad_gate = grad_output * up * silu_derivative
        grad_up = grad_output * silu_gate
        return grad_gate, grad_up, None


def _validate_triton_inputs(gate: Tensor, up: Tensor) -> None:
    """Launch constraints of the fused path (reference swiglu.py:84-94)."""

    require_hip(TritonSwiGLUUnavailable, "SwiGLU", gate, up)
    if gate.shape != up.shape or not gate.is_contiguous() or not up.is_contiguous():
        raise TritonSwiGLUUnavailable("HIP SwiGLU requires matching contiguous inputs.")
    if gate.dtype != up.dtype or gate.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TritonSwiGLUUnavailable("HIP SwiGLU requires float32, float16 or bfloat16 inputs of one dtype.")


def triton_swiglu(gate: Tensor, up: Tensor) -> Tensor:
    """Fused SwiGLU activation (HIP forward and backward)."""

    _validate_triton_inputs(gate, up)
    return _SwiGLUAutogradFunction.apply(gate, up, True)


def swiglu_with_pytorch_forward(gate: Tensor, up: Tensor) -> Tensor:
    """The reference's CPU-verifiable entry point (swiglu.py:104-107)."""

    return _SwiGLUAutogradFunction.apply(gate, up, False)
