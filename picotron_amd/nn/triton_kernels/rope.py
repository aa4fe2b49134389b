"""Fused rotary embedding (forward and backward) on gfx950 behind picotron's Triton-RoPE
surface.

Drop-in for ``picotron.nn.triton_kernels.rope`` (reference
src/picotron/nn/triton_kernels/rope.py).  The reference kernel is forward-only: it raises
when autograd is recording and needs contiguous ``(batch, heads, seq, head_dim)`` input
with interleaved pairs.  Here the rotation is an autograd Function whose backward is the
inverse rotation (``pt_rope(..., inverse=1)``); it accepts strided views (such as the
``(B, S, H, D)``-memory transpose that attention produces), both the interleaved and the
rotate-half layouts, and query + key in one launch.  Angle tables are fp32.
"""

from __future__ import annotations

import torch
from torch import Tensor

from picotron_amd import ops
from picotron_amd.nn.triton_kernels._gate import require_hip


class TritonRoPEUnavailable(RuntimeError):
    """Raised when the fused (HIP) RoPE path cannot safely run."""


class _RoPEFunction(torch.autograd.Function):
    """Rotate one or two (B, H, S, D) views by fp32 angle tables (by minus the angles when
    ``inverse``); the backward is the rotation the other way."""

    @staticmethod
    def forward(ctx, layout: str, inverse: bool, cosine: Tensor, sine: Tensor, *states: Tensor):  # type: ignore[override]
        ctx.layout = layout
        ctx.inverse = inverse
        ctx.save_for_backward(cosine, sine)
        ctx.count = len(states)
        out0, out1 = ops.rope(
            states[0], cosine, sine, layout=layout, inverse=inverse,
            x1=states[1] if len(states) > 1 else None,
        )
        return (out0,) if out1 is None else (out0, out1)

    @staticmethod
    def backward(ctx, *grads: Tensor):  # type: ignore[override]
        cosine, sine = ctx.saved_tensors
        present = [i for i, g in enumerate(grads) if g is not None and ctx.needs_input_grad[4 + i]]
        results: list[Tensor | None] = [None] * ctx.count
        if present:
            g = [_last_dim_contiguous(grads[i]) for i in present]
            if torch.is_grad_enabled() and not ops._compiling():
                # create_graph=True: the backward rotation as this Function again, so that
                # autograd can differentiate it to any order
                d = _RoPEFunction.apply(ctx.layout, not ctx.inverse, cosine, sine, *g)
                d0, d1 = d[0], (d[1] if len(d) > 1 else None)
            else:
                d0, d1 = ops.rope(
                    g[0], cosine, sine, layout=ctx.layout, inverse=not ctx.inverse,
                    x1=g[1] if len(g) > 1 else None,
                )
            results[present[0]] = d0
            if len(present) > 1:
                results[present[1]] = d1
        return (None, None, None, None, *results)


def _last_dim_contiguous(t: Tensor) -> Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _validate(states: list[Tensor], cosine: Tensor, sine: Tensor) -> None:
    require_hip(TritonRoPEUnavailable, "RoPE", *states, cosine, sine)
    head_dim = states[0].size(-1)
    for s in states:
        if (
            s.ndim != 4
            or s.size(-1) != head_dim
            or s.stride(-1) != 1
            or s.dtype not in (torch.float32, torch.float16, torch.bfloat16)
            or s.dtype != states[0].dtype
        ):
            raise TritonRoPEUnavailable(
                "HIP RoPE requires 4-D (batch, heads, seq, head_dim) float states with a "
                "contiguous head_dim."
            )
    if (
        cosine.ndim != 2
        or cosine.shape != sine.shape
        or cosine.size(-1) * 2 != head_dim
        or cosine.size(0) < states[0].size(-2)
    ):
        raise TritonRoPEUnavailable("HIP RoPE requires [seq, head_dim/2] cosine/sine tables.")
    if len(states) == 2 and (
        states[1].size(0) != states[0].size(0) or states[1].size(-2) != states[0].size(-2)
    ):
        raise TritonRoPEUnavailable("RoPE query and key must share batch and sequence sizes.")


def triton_apply_rotary_embedding(
    states: Tensor, cosine: Tensor, sine: Tensor, *, layout: str = "interleaved"
) -> Tensor:
    """Rotate ``(batch, heads, sequence, head_dim)`` states (reference rope.py:52-91).

    Unlike the reference kernel this works with autograd enabled and on strided views.
    Tables of any float dtype are used in fp32.
    """

    _validate([states], cosine, sine)
    return _RoPEFunction.apply(layout, False, cosine.float(), sine.float(), states)[0]


def triton_apply_rotary_embedding_pair(
    query: Tensor, key: Tensor, cosine: Tensor, sine: Tensor, *, layout: str = "interleaved"
) -> tuple[Tensor, Tensor]:
    """Rotate query and key (GQA: head counts may differ) in one kernel launch."""

    _validate([query, key], cosine, sine)
    out_q, out_k = _RoPEFunction.apply(layout, False, cosine.float(), sine.float(), query, key)
    return out_q, out_k
