"""Fused cross-entropy forward + backward on gfx950 behind picotron's Triton-CE surface.

Drop-in for ``picotron.nn.triton_kernels.cross_entropy`` (reference
src/picotron/nn/triton_kernels/cross_entropy.py).  The reference kernel is inference-only,
2-D, vocab <= 65536, without ``ignore_index``, and checks targets with a host sync; its
callers fall back to ``F.cross_entropy``.  Here ``triton_cross_entropy`` returns the same
value as ``F.cross_entropy(logits, targets)`` (mean over targets != -100, fp32) and, when
the logits require grad, writes d(loss)/d(logits) during the forward, into the logits'
storage or into a new gradient buffer (one HBM read of the logits and one write of the
gradient in either case).  The backward only rescales by the incoming gradient, on device,
and skips even that when it is exactly 1.

In-place contract of ``triton_cross_entropy`` (default ``inplace=True``): after a
grad-enabled call the logits tensor holds the gradient, not the logits.  Its autograd
version counter is bumped, so any other graph node that saved those logits fails loudly at
backward instead of reading wrong values; a plain read of the tensor after the loss (metrics,
logging) would see the gradient.  ``inplace=False`` leaves the logits untouched: the kernel
reads them and writes the gradient into a new buffer of their layout, at the same cost as in
place.  It is the default of ``CrossEntropyWithFallback``, the drop-in for
``F.cross_entropy``.  Logits whose rows overlap in memory (e.g. an expanded tensor) are
refused when the gradient would be written into them (out of place they get a private copy).
fp16 logits keep their values until the backward, which writes
(softmax - onehot) * grad_output / n_valid, rounded to fp16 once, over them (in place) or
into a new buffer from the saved logits: the loss scale of fp16 training arrives only with
the backward, and softmax / n_valid would mostly be below fp16's smallest subnormal.  A
gradient written by the forward is consumed by the backward, so a second backward through
the same graph raises.

The train loop's own call, ``F.cross_entropy(logits[:, :-1, :].transpose(1, 2),
input_ids[:, 1:])`` (reference src/picotron/training/train_loop.py:141-144), passed unchanged
through ``CrossEntropyWithFallback`` (out of place), is recognised by the view's geometry and
computed on the view's base: the backward then returns the base's gradient directly, so
autograd's slice backward (a zero-filled tensor of the base's size and a copy into it) does
not run.

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


def _gradient_target(logits: Tensor, write_grad: bool, inplace: bool,
                     class_dim: int) -> tuple[Tensor, Tensor | None]:
    """(buffer the kernel reads, separate gradient buffer or None).  In place (or without a
    gradient, or fp16, whose forward writes none) the kernel works on the logits themselves;
    otherwise the gradient goes to a new buffer of the logits' layout and the logits are only
    read.  Logits whose rows overlap (an expanded tensor) get a private copy, written in place."""

    buffer = logits.detach()
    if not write_grad or inplace or logits.dtype == torch.float16:
        return buffer, None
    grad = ops.ce_grad_buffer(buffer, class_dim)
    if grad is None:
        return buffer.clone(), None
    return buffer, grad


def _keep(ctx, logits: Tensor, buffer: Tensor, grad: Tensor | None, inplace: bool, ws: Tensor,
          targets: Tensor, ignore_index: int, class_dim: int) -> None:
    if inplace:
        torch.autograd.graph.increment_version(logits)
    ctx.deferred = logits.dtype == torch.float16 and not inplace
    if ctx.deferred:
        # fp16 out of place: the backward computes the gradient from the logits (saved with
        # their version, so a later in-place change of them is caught) into a new buffer
        ctx.save_for_backward(logits)
        ctx.grad_buffer = None
    else:
        ctx.grad_buffer = grad if grad is not None else buffer
    ctx.class_dim = class_dim
    ctx.workspace = ws
    ctx.targets = targets
    ctx.ignore_index = ignore_index


def _take(ctx) -> tuple[Tensor, Tensor | None]:
    """(gradient buffer, logits to compute it from or None) for the backward."""

    if ctx.deferred:
        (logits,) = ctx.saved_tensors
        logits = logits.detach()
        grad = ops.ce_grad_buffer(logits, ctx.class_dim)
        if grad is None:
            return logits.clone(), None
        return grad, logits
    grad = ctx.grad_buffer
    if grad is None:
        raise RuntimeError(_REPEATED_BACKWARD)
    ctx.grad_buffer = None
    return grad, None


class _FusedCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor, ignore_index: int, inplace: bool):  # type: ignore[override]
        write_grad = ctx.needs_input_grad[0]
        buffer, grad = _gradient_target(logits, write_grad, inplace, 1)
        loss, ws = ops.cross_entropy(buffer, targets, ignore_index, write_grad=write_grad, grad=grad)
        if write_grad:
            _keep(ctx, logits, buffer, grad, inplace, ws, targets, ignore_index, 1)
        return loss

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss: Tensor):  # type: ignore[override]
        grad, src = _take(ctx)
        ops.cross_entropy_scale_grad(grad, ctx.targets, grad_loss, ctx.ignore_index, ctx.workspace,
                                     logits=src)
        return grad, None, None, None


class _FusedShiftedCrossEntropy(torch.autograd.Function):
    """``next_targets``: ``input_ids`` holds the (B, S - 1) targets themselves."""

    @staticmethod
    def forward(ctx, logits: Tensor, input_ids: Tensor, ignore_index: int, inplace: bool,  # type: ignore[override]
                next_targets: bool):
        write_grad = ctx.needs_input_grad[0]
        buffer, grad = _gradient_target(logits, write_grad, inplace, 2)
        loss, ws = ops.cross_entropy_shifted(buffer, input_ids, ignore_index,
                                             write_grad=write_grad, grad=grad,
                                             next_targets=next_targets)
        if write_grad:
            _keep(ctx, logits, buffer, grad, inplace, ws, input_ids, ignore_index, 2)
            ctx.next_targets = next_targets
        return loss

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss: Tensor):  # type: ignore[override]
        grad, src = _take(ctx)
        ops.cross_entropy_shifted_scale_grad(grad, ctx.targets, grad_loss, ctx.ignore_index,
                                             ctx.workspace, logits=src,
                                             next_targets=ctx.next_targets)
        return grad, None, None, None, None


def _train_loop_base(logits: Tensor, targets: Tensor) -> Tensor | None:
    """The (B, S, V) tensor whose ``[:, :-1, :].transpose(1, 2)`` view ``logits`` is (the train
    loop's call, reference src/picotron/training/train_loop.py:141-144), when the gradient of
    the loss will flow to it; else None.  The loss is then computed on the base rows with the
    last position excluded, and the backward returns the gradient of the base directly (its
    last position zero, as autograd's slice backward would leave it) instead of a gradient of
    the view that the slice backward would copy into a zero-filled tensor of the base's size."""

    base = logits._base
    if (base is None or logits.dim() != 3 or base.dim() != 3 or targets.dim() != 2
            or not base.requires_grad or logits.grad_fn is None):
        return None
    b, s, v = base.shape
    if s < 2 or tuple(logits.shape) != (b, v, s - 1) or tuple(targets.shape) != (b, s - 1):
        return None
    if base.stride(2) != 1 or logits.stride() != (base.stride(0), base.stride(2), base.stride(1)):
        return None
    if logits.storage_offset() != base.storage_offset():
        return None
    return base


def _check_targets(targets: Tensor, vocab: int, ignore_index: int) -> None:
    if os.environ.get(_CHECK_ENV, "") not in ("", "0"):
        bad = ((targets < 0) | (targets >= vocab)) & (targets != ignore_index)
        if bool(bad.any().item()):
            raise TritonCrossEntropyUnavailable("HIP cross-entropy targets are out of range.")


def _validate(logits: Tensor, targets: Tensor, ignore_index: int, shift: bool,
              grad_in_place: bool, next_targets: bool = False) -> None:
    require_hip(TritonCrossEntropyUnavailable, "cross-entropy", logits, targets)
    if logits.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TritonCrossEntropyUnavailable("HIP cross-entropy supports float logits only.")
    try:
        if shift:
            b, s, bs, ss, v, _, _ = ops._shifted_desc(logits, targets, next_targets)
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
        _check_targets(targets if next_targets else targets[:, 1:], logits.size(2), ignore_index)
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

    grad_enabled = logits.requires_grad and torch.is_grad_enabled()
    grad_in_place = bool(inplace) and grad_enabled
    if not shift and not inplace and grad_enabled:
        base = _train_loop_base(logits, targets)
        if base is not None:
            _validate(base, targets, ignore_index, True, False, next_targets=True)
            return _FusedShiftedCrossEntropy.apply(base, targets, int(ignore_index), False, True)
    _validate(logits, targets, ignore_index, shift, grad_in_place)
    if shift:
        return _FusedShiftedCrossEntropy.apply(logits, targets, int(ignore_index), bool(inplace),
                                               False)
    return _FusedCrossEntropy.apply(logits, targets, int(ignore_index), bool(inplace))


class CrossEntropyWithFallback:
    """Run the fused cross-entropy when enabled, else (or on failure) ``F.cross_entropy``
    (reference cross_entropy.py:90-109).

    Like ``F.cross_entropy`` it leaves its input alone by default: the fused path then reads
    the logits and writes the gradient into a new buffer (one read and one write in all).
    ``inplace=True`` writes it over the logits themselves, which saves that buffer's memory,
    for callers that do not read the logits after the loss -- the train loop
    (train_loop.py:136-160) is one: its logits feed only the loss."""

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
