"""Fused cross-entropy forward + backward on gfx950 behind picotron's Triton-CE surface.

Drop-in for ``picotron.nn.triton_kernels.cross_entropy`` (reference
src/picotron/nn/triton_kernels/cross_entropy.py).  The reference kernel is inference-only,
2-D, vocab <= 65536, without ``ignore_index``, and checks targets with a host sync; its
callers fall back to ``F.cross_entropy``.  Here ``triton_cross_entropy`` returns the same
value as ``F.cross_entropy(logits, targets)`` (mean over targets != -100, fp32) and, when
the logits require grad, writes d(loss)/d(logits) into the logits' storage during the
forward (one HBM read + one write of the logits in total).  The backward only rescales by
the incoming gradient, on device, and skips even that when it is exactly 1.

In-place contract of ``triton_cross_entropy`` (default ``inplace=True``): after a
grad-enabled call the logits tensor holds the gradient, not the logits.  Its autograd
version counter is bumped, so any other graph node that saved those logits fails loudly at
backward instead of reading wrong values; a plain read of the tensor after the loss (metrics,
logging) would see the gradient.  ``inplace=False`` keeps the logits (the gradient then goes
to a copy), and is the default of ``CrossEntropyWithFallback``, the drop-in for
``F.cross_entropy``.  Logits whose rows overlap in memory (e.g. an expanded tensor) are
refused when the gradient would be written into them.  fp16 logits keep their values until
the backward, which writes (softmax - onehot) * grad_output / n_valid over them, rounded to
fp16 once: the loss scale of fp16 training arrives only with the backward, and
softmax / n_valid would mostly be below fp16's smallest subnormal.  The gradient buffer is
consumed by the backward, so a second backward through the same graph raises.

``shift=True`` takes the language model's whole (B, S, V) logits and the (B, S) input ids
and computes the train loop's next-token loss (reference
src/picotron/training/train_loop.py:141-144, ``logits[:, :-1, :].transpose(1, 2)`` against
``input_ids[:, 1:]``) without the slice: the gradient then covers the whole logits buffer
(last position zero), so autograd skips the slice backward's full-size zero fill and copy.
"""

from __future__ import annotations

import os
import warnings

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable
from torch.nn import functional as F

from picotron_amd import ops
from picotron_amd.nn.triton_kernels._gate import require_hip

IGNORE_INDEX = -100
_CHECK_ENV = "PICOTRON_HIP_CE_CHECK"


class TritonCrossEntropyUnavailable(RuntimeError):
    """Raised when the fused (HIP) cross-entropy path cannot safely run."""


_REPEATED_BACKWARD = (
    "the fused cross-entropy's gradient buffer was consumed by an earlier backward through "
    "this graph (retain_graph=True); backpropagate through the loss once, or compute it with "
    "F.cross_entropy"
)


class _FusedCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor, ignore_index: int, inplace: bool):  # type: ignore[override]
        write_grad = ctx.needs_input_grad[0]
        buffer = logits.detach()
        if write_grad and not inplace:
            buffer = buffer.clone()
        loss, ws = ops.cross_entropy(buffer, targets, ignore_index, write_grad=write_grad)
        if write_grad:
            if inplace:
                torch.autograd.graph.increment_version(logits)
            ctx.grad_buffer = buffer
            ctx.workspace = ws
            ctx.targets = targets
            ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss: Tensor):  # type: ignore[override]
        grad = getattr(ctx, "grad_buffer", None)
        if grad is None:
            raise RuntimeError(_REPEATED_BACKWARD)
        ops.cross_entropy_scale_grad(grad, ctx.targets, grad_loss, ctx.ignore_index, ctx.workspace)
        ctx.grad_buffer = None
        return grad, None, None, None


class _FusedShiftedCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, input_ids: Tensor, ignore_index: int, inplace: bool):  # type: ignore[override]
        write_grad = ctx.needs_input_grad[0]
        buffer = logits.detach()
        if write_grad and not inplace:
            buffer = buffer.clone()
        loss, ws = ops.cross_entropy_shifted(buffer, input_ids, ignore_index, write_grad=write_grad)
        if write_grad:
            if inplace:
                torch.autograd.graph.increment_version(logits)
            ctx.grad_buffer = buffer
            ctx.workspace = ws
            ctx.input_ids = input_ids
            ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss: Tensor):  # type: ignore[override]
        grad = getattr(ctx, "grad_buffer", None)
        if grad is None:
            raise RuntimeError(_REPEATED_BACKWARD)
        ops.cross_entropy_shifted_scale_grad(grad, ctx.input_ids, grad_loss, ctx.ignore_index,
                                             ctx.workspace)
        ctx.grad_buffer = None
        return grad, None, None, None


def _check_targets(targets: Tensor, vocab: int, ignore_index: int) -> None:
    if os.environ.get(_CHECK_ENV, "") not in ("", "0"):
        bad = ((targets < 0) | (targets >= vocab)) & (targets != ignore_index)
        if bool(bad.any().item()):
            raise TritonCrossEntropyUnavailable("HIP cross-entropy targets are out of range.")


def _validate(logits: Tensor, targets: Tensor, ignore_index: int, shift: bool,
              grad_in_place: bool) -> None:
    require_hip(TritonCrossEntropyUnavailable, "cross-entropy", logits, targets)
    if logits.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TritonCrossEntropyUnavailable("HIP cross-entropy supports float logits only.")
    try:
        if shift:
            b, s, bs, ss, v, _, _ = ops._shifted_desc(logits, targets)
            rows = [(b, bs), (s, ss)]
        else:
            outer, inner, os_, is_, v = ops.ce_rows(logits)
            ops.ce_target_strides(targets, outer, inner)
            rows = [(outer, os_), (inner, is_)]
    except ValueError as error:
        raise TritonCrossEntropyUnavailable(f"HIP cross-entropy: {error}.") from error
    if grad_in_place and not ops.rows_disjoint(rows, v):
        raise TritonCrossEntropyUnavailable(
            "HIP cross-entropy: logits rows overlap in memory, so the gradient cannot be "
            "written into them; pass inplace=False.")
    if shift:
        _check_targets(targets[:, 1:], logits.size(2), ignore_index)
    else:
        _check_targets(targets, logits.size(1), ignore_index)


def triton_cross_entropy(
    logits: Tensor,
    targets: Tensor,
    *,
    ignore_index: int = IGNORE_INDEX,
    inplace: bool = True,
    shift: bool = False,
) -> Tensor:
    """Mean cross-entropy over targets != ignore_index as an fp32 scalar.

    ``logits`` is (N, C) or (N, C, d) with a contiguous class dimension (such as the
    ``logits[:, :-1, :].transpose(1, 2)`` view of the train loop); ``targets`` is (N,) or
    (N, d) int64.  With ``shift=True``, ``logits`` is the model's (B, S, V) output and
    ``targets`` the (B, S) input ids: the loss is that of ``logits[:, :-1, :]`` against
    ``targets[:, 1:]``.  A non-ignored target outside [0, C) gives a NaN loss (set
    PICOTRON_HIP_CE_CHECK=1 to raise instead, at the cost of a host sync).
    """

    grad_in_place = bool(inplace) and logits.requires_grad and torch.is_grad_enabled()
    _validate(logits, targets, ignore_index, shift, grad_in_place)
    fn = _FusedShiftedCrossEntropy if shift else _FusedCrossEntropy
    return fn.apply(logits, targets, int(ignore_index), bool(inplace))


class CrossEntropyWithFallback:
    """Run the fused cross-entropy when enabled, else (or on failure) ``F.cross_entropy``
    (reference cross_entropy.py:90-109).

    Like ``F.cross_entropy`` it leaves its input alone by default: the fused path then
    writes the gradient into a copy of the logits.  ``inplace=True`` writes it into the
    logits themselves (one read and one write of the logits in all), for callers that do not
    read the logits after the loss -- the train loop (train_loop.py:136-160) is one: its
    logits feed only the loss."""

    def __init__(self, *, use_triton: bool = False, inplace: bool = False) -> None:
        self.use_triton = use_triton
        self.inplace = inplace
        self._fallback_warned = False

    def __call__(self, logits: Tensor, targets: Tensor, *, shift: bool = False) -> Tensor:
        """``shift=True``: ``logits`` (B, S, V) and ``targets`` the (B, S) input ids; the
        loss is the train loop's ``F.cross_entropy(logits[:, :-1, :].transpose(1, 2),
        targets[:, 1:])`` (reference train_loop.py:141-144)."""

        if self.use_triton:
            try:
                return triton_cross_entropy(logits, targets, shift=shift, inplace=self.inplace)
            except Exception as error:
                if not self._fallback_warned:
                    warnings.warn(
                        f"Triton cross-entropy unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._fallback_warned = True
        if shift:
            return F.cross_entropy(logits[:, :-1, :].transpose(1, 2), targets[:, 1:])
        return F.cross_entropy(logits, targets)
