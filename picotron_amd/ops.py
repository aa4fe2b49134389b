"""Tensor-level launchers for the HIP kernels: shape/stride checks, output allocation,
and the ctypes call on the caller's current HIP stream.

These functions never fall back to PyTorch arithmetic: if the library is missing they
raise :class:`picotron_amd._lib.HipLibraryUnavailable`, and if an entry point rejects its
arguments they raise :class:`picotron_amd._lib.HipKernelError`.  The autograd Functions
in :mod:`picotron_amd.nn.triton_kernels` are built on them.
"""

from __future__ import annotations

import ctypes
import functools

import numpy as np
import torch
from torch import Tensor

from picotron_amd import _lib

_DTYPE_CODES = {
    torch.float32: _lib.PT_FLOAT32,
    torch.float16: _lib.PT_FLOAT16,
    torch.bfloat16: _lib.PT_BFLOAT16,
}

LAYOUTS = {"interleaved": 0, "rotate_half": 1}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The device's current HIP stream as an integer handle (torch's raw-stream query when
    present: it skips building a Stream object on every launch)."""

    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


@functools.lru_cache(maxsize=256)
def _rmsnorm_ws_bytes(rows: int, cols: int, code: int) -> int:
    return int(_lib.lib().pt_rmsnorm_bwd_workspace_bytes(rows, cols, code))


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _compiling() -> bool:
    """True while torch.compile traces: the launchers then record themselves as the custom
    ops registered at the end of this module (opaque to the compiler, with fake
    implementations for shape propagation) instead of calling the library; at run time the
    compiled graph calls those ops, which call the launchers eagerly."""

    return torch.compiler.is_compiling()


@functools.lru_cache(maxsize=None)
def device_supported(index: int) -> bool:
    """True if CUDA/HIP device ``index`` is a gfx950 GPU the library was built for."""

    return bool(_lib.lib().pt_device_supported(index))


def _check_cuda(*tensors: Tensor) -> torch.device:
    device = tensors[0].device
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("HIP kernels need tensors on a GPU device")
        if t.device != device:
            raise ValueError("all tensors must be on the same device")
    return device


# ------------------------------------------------------------------ RMSNorm


def _as_rows(t: Tensor, cols: int) -> Tensor:
    """(rows, cols) view of ``t`` whose last dim is contiguous; copies only if needed."""

    if t.dim() == 2 and t.size(1) == cols and (t.stride(1) == 1 or cols == 1):
        return t
    flat = t.reshape(-1, cols)
    if flat.size(0) > 1 and flat.stride(1) != 1:
        flat = flat.contiguous()
    return flat


def rmsnorm_fwd(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dim; returns (y, rstd fp32)."""

    if _compiling():
        return torch.ops.picotron_amd.rmsnorm_fwd(x, weight, float(eps))
    device = _check_cuda(x, weight)
    cols = x.size(-1)
    if weight.dim() != 1 or weight.numel() != cols:
        raise ValueError("RMSNorm weight must be 1-D with hidden-size elements")
    weight = weight.contiguous()
    x2 = _as_rows(x, cols)
    rows = x2.size(0)
    y = torch.empty(x.shape, dtype=x.dtype, device=device)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=device)
    y2 = y.view(-1, cols)
    _lib.call(
        "pt_rmsnorm_fwd",
        x2.data_ptr(), x2.stride(0) if rows > 1 else cols, weight.data_ptr(), y2.data_ptr(), cols,
        rstd.data_ptr(), rows, cols, float(eps), dtype_code(x.dtype), dtype_code(weight.dtype),
        _stream(device),
    )
    return y, rstd


def rmsnorm_bwd(
    dy: Tensor,
    x: Tensor,
    weight: Tensor,
    rstd: Tensor,
    need_dx: bool = True,
    need_dw: bool = True,
) -> tuple[Tensor | None, Tensor | None]:
    """Gradients of RMSNorm w.r.t. x (x's dtype) and weight (weight's dtype)."""

    if _compiling():
        dx, dw = torch.ops.picotron_amd.rmsnorm_bwd(dy, x, weight, rstd)
        return (dx if need_dx else None), (dw if need_dw else None)
    device = _check_cuda(dy, x, weight, rstd)
    cols = x.size(-1)
    if dy.dtype != x.dtype:
        dy = dy.to(x.dtype)
    weight = weight.contiguous()
    rstd = rstd.contiguous()
    x2 = _as_rows(x, cols)
    dy2 = _as_rows(dy, cols)
    rows = x2.size(0)
    if rstd.numel() != rows or rstd.dtype != torch.float32:
        raise ValueError("rstd must hold one fp32 value per row")
    dx = torch.empty(x.shape, dtype=x.dtype, device=device) if need_dx else None
    dw = torch.empty(cols, dtype=weight.dtype, device=device) if need_dw else None
    ws = None
    ws_bytes = 0
    if need_dw:
        ws_bytes = _rmsnorm_ws_bytes(rows, cols, dtype_code(x.dtype))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    if not need_dx and not need_dw:
        return None, None
    _lib.call(
        "pt_rmsnorm_bwd",
        dy2.data_ptr(), dy2.stride(0) if rows > 1 else cols, x2.data_ptr(),
        x2.stride(0) if rows > 1 else cols, weight.data_ptr(), rstd.data_ptr(), _ptr(dx), cols,
        _ptr(dw), _ptr(ws), ws_bytes, rows, cols, dtype_code(x.dtype), dtype_code(weight.dtype),
        _stream(device),
    )
    return dx, dw


def residual_rmsnorm_fwd(
    x: Tensor, residual: Tensor, weight: Tensor, eps: float
) -> tuple[Tensor, Tensor, Tensor]:
    """h = x + residual (rounded to x's dtype) and y = RMSNorm(h) in one pass; returns
    (h, y, rstd fp32)."""

    if _compiling():
        return torch.ops.picotron_amd.residual_rmsnorm_fwd(x, residual, weight, float(eps))
    device = _check_cuda(x, residual, weight)
    cols = x.size(-1)
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError("residual must match x in shape and dtype")
    if weight.dim() != 1 or weight.numel() != cols:
        raise ValueError("RMSNorm weight must be 1-D with hidden-size elements")
    weight = weight.contiguous()
    x2 = _as_rows(x, cols)
    r2 = _as_rows(residual, cols)
    rows = x2.size(0)
    h = torch.empty(x.shape, dtype=x.dtype, device=device)
    y = torch.empty(x.shape, dtype=x.dtype, device=device)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=device)
    _lib.call(
        "pt_residual_rmsnorm_fwd",
        x2.data_ptr(), x2.stride(0) if rows > 1 else cols, r2.data_ptr(),
        r2.stride(0) if rows > 1 else cols, weight.data_ptr(), h.data_ptr(), cols, y.data_ptr(), cols,
        rstd.data_ptr(), rows, cols, float(eps), dtype_code(x.dtype), dtype_code(weight.dtype),
        _stream(device),
    )
    return h, y, rstd


def residual_rmsnorm_bwd(
    dy: Tensor,
    dh_in: Tensor | None,
    h: Tensor,
    weight: Tensor,
    rstd: Tensor,
    need_dw: bool = True,
    out: Tensor | None = None,
) -> tuple[Tensor, Tensor | None]:
    """dh = RMSNorm-backward(dy) + dh_in (in h's dtype) and the weight gradient.  ``out``
    (may be ``dh_in`` itself) receives dh when given."""

    if _compiling() and out is None:
        dh, dw = torch.ops.picotron_amd.residual_rmsnorm_bwd(dy, dh_in, h, weight, rstd)
        return dh, (dw if need_dw else None)
    device = _check_cuda(dy, h, weight, rstd)
    cols = h.size(-1)
    if dy.dtype != h.dtype:
        dy = dy.to(h.dtype)
    weight = weight.contiguous()
    rstd = rstd.contiguous()
    h2 = _as_rows(h, cols)
    dy2 = _as_rows(dy, cols)
    rows = h2.size(0)
    if rstd.numel() != rows or rstd.dtype != torch.float32:
        raise ValueError("rstd must hold one fp32 value per row")
    d2 = None
    if dh_in is not None:
        if dh_in.shape != h.shape:
            raise ValueError("dh_in must match h")
        if dh_in.dtype != h.dtype:
            dh_in = dh_in.to(h.dtype)
        d2 = _as_rows(dh_in, cols)
    if out is None:
        out = torch.empty(h.shape, dtype=h.dtype, device=device)
    elif out.shape != h.shape or out.dtype != h.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor like h")
    dw = torch.empty(cols, dtype=weight.dtype, device=device) if need_dw else None
    ws, ws_bytes = None, 0
    if need_dw:
        ws_bytes = _rmsnorm_ws_bytes(rows, cols, dtype_code(h.dtype))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    _lib.call(
        "pt_residual_rmsnorm_bwd",
        dy2.data_ptr(), dy2.stride(0) if rows > 1 else cols, _ptr(d2),
        (d2.stride(0) if rows > 1 else cols) if d2 is not None else 0, h2.data_ptr(),
        h2.stride(0) if rows > 1 else cols, weight.data_ptr(), rstd.data_ptr(), out.data_ptr(), cols,
        _ptr(dw), _ptr(ws), ws_bytes, rows, cols, dtype_code(h.dtype), dtype_code(weight.dtype),
        _stream(device),
    )
    return out, dw


# ------------------------------------------------------------------ SwiGLU


def _flat(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


def swiglu_fwd(gate: Tensor, up: Tensor) -> Tensor:
    """silu(gate) * up, elementwise, in gate's dtype."""

    if _compiling():
        return torch.ops.picotron_amd.swiglu_fwd(gate, up)
    device = _check_cuda(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("SwiGLU gate and up must match in shape and dtype")
    gate, up = _flat(gate), _flat(up)
    out = torch.empty_like(gate)
    _lib.call(
        "pt_swiglu_fwd", gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
        dtype_code(gate.dtype), _stream(device),
    )
    return out


def swiglu_bwd(
    dout: Tensor, gate: Tensor, up: Tensor, need_dgate: bool = True, need_dup: bool = True
) -> tuple[Tensor | None, Tensor | None]:
    if _compiling():
        dg, du = torch.ops.picotron_amd.swiglu_bwd(dout, gate, up)
        return (dg if need_dgate else None), (du if need_dup else None)
    device = _check_cuda(dout, gate, up)
    if dout.dtype != gate.dtype:
        dout = dout.to(gate.dtype)
    dout, gate, up = _flat(dout), _flat(gate), _flat(up)
    dg = torch.empty_like(gate) if need_dgate else None
    du = torch.empty_like(up) if need_dup else None
    _lib.call(
        "pt_swiglu_bwd", dout.data_ptr(), gate.data_ptr(), up.data_ptr(), _ptr(dg), _ptr(du),
        gate.numel(), dtype_code(gate.dtype), _stream(device),
    )
    return dg, du


# ------------------------------------------------------------------ RoPE


def _rope_desc(x: Tensor, y: Tensor) -> ctypes.Array:
    b, h, s, _ = x.shape
    return (ctypes.c_int64 * 9)(
        b, h, s, x.stride(0), x.stride(1), x.stride(2), y.stride(0), y.stride(1), y.stride(2)
    )


def rope(
    x0: Tensor,
    cos: Tensor,
    sin: Tensor,
    *,
    layout: str = "interleaved",
    inverse: bool = False,
    x1: Tensor | None = None,
) -> tuple[Tensor, Tensor | None]:
    """Rotate (batch, heads, seq, head_dim) views x0 (and x1) by the angle tables.

    ``cos``/``sin`` are fp32 ``[>= seq, head_dim/2]`` tables; row ``s`` is position ``s``.
    Outputs are new tensors with the inputs' logical shape and memory layout.
    """

    if _compiling():
        if x1 is None:
            return torch.ops.picotron_amd.rope(x0, cos, sin, layout, bool(inverse)), None
        y0, y1 = torch.ops.picotron_amd.rope_pair(x0, x1, cos, sin, layout, bool(inverse))
        return y0, y1
    device = _check_cuda(x0, cos, sin) if x1 is None else _check_cuda(x0, x1, cos, sin)
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(LAYOUTS)}")
    tensors = [x0] if x1 is None else [x0, x1]
    head_dim = x0.size(-1)
    for t in tensors:
        if t.dim() != 4 or t.size(-1) != head_dim or t.stride(-1) != 1:
            raise ValueError("RoPE states must be 4-D (batch, heads, seq, head_dim), head_dim contiguous")
        if t.dtype != x0.dtype:
            raise ValueError("query and key must share a dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError("RoPE tables must be fp32")
    cos = cos.contiguous()
    sin = sin.contiguous()
    if cos.dim() != 2 or cos.shape != sin.shape or cos.size(1) * 2 != head_dim:
        raise ValueError("RoPE tables must be [seq, head_dim/2]")
    # empty_like keeps the input's stride order (dense inputs), so a (B,S,H,D)-memory view
    # comes back with the same memory layout.
    outs = [torch.empty_like(t) for t in tensors]
    descs = [_rope_desc(t, o) for t, o in zip(tensors, outs)]
    _lib.call(
        "pt_rope",
        x0.data_ptr(), outs[0].data_ptr(), descs[0],
        None if x1 is None else x1.data_ptr(), None if x1 is None else outs[1].data_ptr(),
        None if x1 is None else descs[1],
        head_dim, cos.data_ptr(), sin.data_ptr(), cos.size(0), LAYOUTS[layout], int(inverse),
        dtype_code(x0.dtype), _stream(device),
    )
    return outs[0], (outs[1] if x1 is not None else None)


# ------------------------------------------------------------------ cross-entropy


def ce_rows(logits: Tensor) -> tuple[int, int, int, int, int]:
    """(outer, inner, outer_stride, inner_stride, vocab) of a (N, V) or (B, V, S) input
    whose class dimension (dim 1) is contiguous."""

    if logits.dim() == 2:
        n, v = logits.shape
        if logits.stride(1) != 1 and v > 1:
            raise ValueError("cross-entropy logits need a contiguous class dimension")
        return n, 1, logits.stride(0), 0, v
    if logits.dim() == 3:
        b, v, s = logits.shape
        if logits.stride(1) != 1 and v > 1:
            raise ValueError("cross-entropy logits need a contiguous class dimension")
        return b, s, logits.stride(0), logits.stride(2), v
    raise ValueError("cross-entropy logits must be (N, C) or (N, C, d)")


def rows_disjoint(sizes_strides: list[tuple[int, int]], row_len: int) -> bool:
    """True if rows of ``row_len`` contiguous elements, one per index of the given
    (size, stride) dimensions, never share an element (sufficient test: each stride, in
    increasing order, clears the extent spanned by the dimensions below it)."""

    extent = row_len  # elements spanned by one index of every dimension seen so far
    for stride, size in sorted((abs(st), sz) for sz, st in sizes_strides if sz > 1):
        if stride < extent:
            return False
        extent += stride * (size - 1)
    return True


def ce_target_strides(targets: Tensor, outer: int, inner: int) -> tuple[int, int]:
    if targets.dtype != torch.long:
        raise ValueError("cross-entropy targets must be int64")
    if targets.dim() == 1 and inner == 1:
        if targets.numel() != outer:
            raise ValueError("targets must have one entry per row")
        return targets.stride(0), 0
    if targets.dim() == 2 and tuple(targets.shape) == (outer, inner):
        return targets.stride(0), targets.stride(1)
    raise ValueError("targets shape does not match the logits")


def ce_grad_buffer(logits: Tensor, class_dim: int = 1) -> Tensor | None:
    """An uninitialised tensor of the logits' shape and strides whose data starts in the same
    128-byte phase as the logits', so that every gradient row starts in the phase of its
    logits row: the fused kernels require the same 16-byte phase of a separate gradient, and
    split rows at the logits' 128-byte cache lines, which are then the gradient's lines too
    (and the result bitwise the in-place call's).  ``class_dim``: the contiguous class
    dimension, 1 for (N, C) and (N, C, d) inputs, 2 for the shifted (B, S, V) form.  None when
    the logits rows overlap in memory (an expanded tensor)."""

    dims = list(zip(logits.shape, logits.stride()))
    rows = [d for i, d in enumerate(dims) if i != class_dim]
    if not rows_disjoint(rows, logits.size(class_dim)):
        return None
    if logits.numel() == 0:
        return torch.empty_like(logits)
    span = 1 + sum((n - 1) * st for n, st in dims)
    per_line = 128 // logits.element_size()
    flat = torch.empty(span + per_line, dtype=logits.dtype, device=logits.device)
    offset = ((logits.data_ptr() - flat.data_ptr()) % 128) // logits.element_size()
    return flat.as_strided(logits.shape, logits.stride(), flat.storage_offset() + offset)


def cross_entropy(
    logits: Tensor, targets: Tensor, ignore_index: int = -100, write_grad: bool = False,
    grad: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Mean cross-entropy (fp32 scalar tensor) over targets != ignore_index.

    With ``write_grad`` (fp32 and bf16) d(loss)/d(logits) is written in the same pass: into
    ``grad`` when given (the logits' shape, rows in the logits rows' 16-byte phase, e.g. from
    :func:`ce_grad_buffer`; the logits are only read), else over the logits in place.  fp16
    writes its gradient in :func:`cross_entropy_scale_grad`.
    Returns (loss, workspace); the workspace holds the status word (bit 0: a target out
    of range), readable with :func:`cross_entropy_status`.
    """

    device = _check_cuda(logits, targets)
    outer, inner, os_, is_, vocab = ce_rows(logits)
    tos, tis = ce_target_strides(targets, outer, inner)
    gos = gis = 0
    if grad is not None:
        if grad.shape != logits.shape or grad.dtype != logits.dtype or grad.device != logits.device:
            raise ValueError("the gradient buffer must match the logits")
        _, _, gos, gis, _ = ce_rows(grad)
        if write_grad and not rows_disjoint([(outer, gos), (inner, gis)], vocab):
            raise ValueError("cross-entropy gradient rows overlap in memory")
    elif write_grad and not rows_disjoint([(outer, os_), (inner, is_)], vocab):
        raise ValueError("cross-entropy logits rows overlap in memory; the gradient cannot be "
                         "written into them")
    rows = outer * inner
    ws_bytes = _lib.lib().pt_cross_entropy_workspace_bytes(rows)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    loss = torch.empty((), dtype=torch.float32, device=device)
    _lib.call(
        "pt_cross_entropy",
        logits.data_ptr(), outer, inner, os_, is_, vocab, targets.data_ptr(), tos, tis,
        int(ignore_index), loss.data_ptr(), int(write_grad), _ptr(grad), gos, gis, ws.data_ptr(),
        ws_bytes, dtype_code(logits.dtype), _stream(device),
    )
    return loss, ws


def cross_entropy_status(ws: Tensor) -> int:
    """Status word of a cross-entropy workspace (synchronises with the device)."""

    return int(ws[8:12].view(torch.int32).item())


def cross_entropy_scale_grad(
    dlogits: Tensor, targets: Tensor, grad_output: Tensor, ignore_index: int = -100,
    workspace: Tensor | None = None, logits: Tensor | None = None,
) -> None:
    """dlogits *= grad_output in place (skipped on device when grad_output == 1).  For fp16
    the forward left the logits unchanged and this call writes the gradient,
    (softmax - onehot) * grad_output / n_valid rounded once, from the row log-sum-exps and
    n_valid in ``workspace`` (the forward's): computed from ``logits`` into ``dlogits`` (rows
    in the same 16-byte phase) when ``logits`` is given, else over ``dlogits`` in place."""

    device = _check_cuda(dlogits, targets, grad_output)
    outer, inner, os_, is_, vocab = ce_rows(dlogits)
    tos, tis = ce_target_strides(targets, outer, inner)
    los = lis = 0
    if logits is not None:
        if logits.shape != dlogits.shape or logits.dtype != dlogits.dtype:
            raise ValueError("logits must match the gradient buffer")
        _, _, los, lis, _ = ce_rows(logits)
    go = grad_output.detach().to(torch.float32).reshape(())
    _lib.call(
        "pt_cross_entropy_scale_grad",
        dlogits.data_ptr(), outer, inner, os_, is_, vocab, targets.data_ptr(), tos, tis,
        int(ignore_index), go.data_ptr(), _ptr(logits), los, lis, _ptr(workspace),
        dtype_code(dlogits.dtype), _stream(device),
    )


def _shifted_desc(logits: Tensor, input_ids: Tensor,
                  next_targets: bool = False) -> tuple[int, int, int, int, int, int, int]:
    """(batch, seq, batch_stride, seq_stride, vocab, ids_batch_stride, ids_seq_stride).
    ``next_targets``: ``input_ids`` holds the targets themselves, (batch, seq - 1), entry
    (b, t) for position t (the train loop's ``input_ids[:, 1:]``)."""

    if logits.dim() != 3:
        raise ValueError("shifted cross-entropy logits must be (batch, seq, vocab)")
    b, s, v = logits.shape
    if logits.stride(2) != 1 and v > 1:
        raise ValueError("cross-entropy logits need a contiguous vocabulary dimension")
    if input_ids.dtype != torch.long:
        raise ValueError("cross-entropy targets must be int64")
    want = (b, s - 1) if next_targets else (b, s)
    if input_ids.dim() != 2 or tuple(input_ids.shape) != want:
        raise ValueError(f"targets must be {want} for (batch, seq, vocab) logits")
    return b, s, logits.stride(0), logits.stride(1), v, input_ids.stride(0), input_ids.stride(1)


def _ids_ptr(input_ids: Tensor, next_targets: bool) -> int:
    """The address the shifted entry points take as input_ids: they read position t's target
    at input_ids + (t + 1) * seq_stride, so targets already shifted by one (entry t for
    position t) are passed as the address one position before them (never dereferenced)."""

    if not next_targets:
        return input_ids.data_ptr()
    return input_ids.data_ptr() - input_ids.stride(1) * input_ids.element_size()


def cross_entropy_shifted(
    logits: Tensor, input_ids: Tensor, ignore_index: int = -100, write_grad: bool = False,
    grad: Tensor | None = None, next_targets: bool = False,
) -> tuple[Tensor, Tensor]:
    """Next-token mean cross-entropy of (B, S, V) logits against input_ids[:, 1:]: equal to
    :func:`cross_entropy` on ``logits[:, :-1, :].transpose(1, 2)``.  With ``write_grad`` the
    gradient covers the whole (B, S, V) buffer (last position zero): into ``grad`` when
    given (as in :func:`cross_entropy`), else over the logits.  ``next_targets``:
    ``input_ids`` is already the (B, S - 1) targets (the train loop's ``input_ids[:, 1:]``)."""

    device = _check_cuda(logits, input_ids)
    b, s, bs, ss, v, ibs, iss = _shifted_desc(logits, input_ids, next_targets)
    gbs = gss = 0
    if grad is not None:
        if grad.shape != logits.shape or grad.dtype != logits.dtype or grad.device != logits.device:
            raise ValueError("the gradient buffer must match the logits")
        gbs, gss = grad.stride(0), grad.stride(1)
        if grad.stride(2) != 1 and v > 1:
            raise ValueError("the gradient buffer needs a contiguous vocabulary dimension")
        if write_grad and not rows_disjoint([(b, gbs), (s, gss)], v):
            raise ValueError("cross-entropy gradient rows overlap in memory")
    elif write_grad and not rows_disjoint([(b, bs), (s, ss)], v):
        raise ValueError("cross-entropy logits rows overlap in memory; the gradient cannot be "
                         "written into them")
    ws_bytes = _lib.lib().pt_cross_entropy_workspace_bytes(b * s)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    loss = torch.empty((), dtype=torch.float32, device=device)
    _lib.call(
        "pt_cross_entropy_shifted",
        logits.data_ptr(), b, s, bs, ss, v, _ids_ptr(input_ids, next_targets), ibs, iss,
        int(ignore_index), loss.data_ptr(), int(write_grad), _ptr(grad), gbs, gss,
        ws.data_ptr(), ws_bytes, dtype_code(logits.dtype), _stream(device),
    )
    return loss, ws


def cross_entropy_shifted_scale_grad(
    dlogits: Tensor, input_ids: Tensor, grad_output: Tensor, ignore_index: int = -100,
    workspace: Tensor | None = None, logits: Tensor | None = None, next_targets: bool = False,
) -> None:
    """dlogits *= grad_output in place for a gradient from :func:`cross_entropy_shifted`
    (fp16: as :func:`cross_entropy_scale_grad`, with the forward's ``workspace``, from
    ``logits`` into ``dlogits`` when ``logits`` is given)."""

    device = _check_cuda(dlogits, input_ids, grad_output)
    b, s, bs, ss, v, ibs, iss = _shifted_desc(dlogits, input_ids, next_targets)
    lbs = lss = 0
    if logits is not None:
        if logits.shape != dlogits.shape or logits.dtype != dlogits.dtype:
            raise ValueError("logits must match the gradient buffer")
        lbs, lss = logits.stride(0), logits.stride(1)
    go = grad_output.detach().to(torch.float32).reshape(())
    _lib.call(
        "pt_cross_entropy_shifted_scale_grad",
        dlogits.data_ptr(), b, s, bs, ss, v, _ids_ptr(input_ids, next_targets), ibs, iss,
        int(ignore_index), go.data_ptr(), _ptr(logits), lbs, lss, _ptr(workspace),
        dtype_code(dlogits.dtype), _stream(device),
    )


# ------------------------------------------------------------------ AdamW


def adamw_block_elems() -> int:
    return int(_lib.lib().pt_adamw_block_elems())


@functools.lru_cache(maxsize=None)
def _adamw_block_elems() -> int:
    return adamw_block_elems()


def adamw_table(
    params: list[Tensor], grads: list[Tensor], exp_avgs: list[Tensor], exp_avg_sqs: list[Tensor]
) -> tuple[Tensor, int]:
    """Host int64 [n, 6] table for :func:`adamw_step` and its total block count."""

    per = _adamw_block_elems()
    rows = []
    first = 0
    for p, g, m, v in zip(params, grads, exp_avgs, exp_avg_sqs):
        n = p.numel()
        if n == 0:
            continue
        rows += (p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), n, first)
        first += (n + per - 1) // per
    table = torch.from_numpy(np.array(rows, dtype=np.int64).reshape(-1, 6))
    return table, first


_MOMENT_ALIGN = 64  # elements: every moment starts 256 bytes apart from the buffer's start


def adamw_moments(params: list[Tensor]) -> list[tuple[Tensor, Tensor]]:
    """Zeroed fp32 (exp_avg, exp_avg_sq) for each of ``params`` (one device, contiguous), as
    views of one allocation: every first moment, then every second moment, each view with its
    parameter's shape and 256-byte aligned.  The two moments of a parameter then lie a fixed
    distance apart inside one allocation; as separate allocations their placement relative to
    each other varies, and the update's four concurrent streams ran up to 8 % slower on some
    placements (1.2e9 parameters: 5.70 against 5.40 ms per step on the same parameters and
    gradients)."""

    offsets = []
    total = 0
    for p in params:
        offsets.append(total)
        total += (p.numel() + _MOMENT_ALIGN - 1) // _MOMENT_ALIGN * _MOMENT_ALIGN
    if not params:
        return []
    buf = torch.zeros(2 * total, dtype=torch.float32, device=params[0].device)
    return [(buf[o:o + p.numel()].view(p.shape), buf[total + o:total + o + p.numel()].view(p.shape))
            for p, o in zip(params, offsets)]


def adamw_step(
    table_device: Tensor,
    total_blocks: int,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: float,
) -> None:
    """One AdamW step over the tensors in a device table built from :func:`adamw_table`."""

    device = _check_cuda(table_device)
    _lib.call(
        "pt_adamw_step",
        table_device.data_ptr(), table_device.size(0), int(total_blocks), float(lr), float(beta1),
        float(beta2), float(eps), float(weight_decay), float(step), _stream(device),
    )


def adamw_step_scaled(
    table_device: Tensor,
    total_blocks: int,
    grad_scale: Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: float,
    write_grad: bool,
) -> None:
    """:func:`adamw_step` with every gradient multiplied by the fp32 device scalar
    ``grad_scale`` as it is read (and stored back when ``write_grad``)."""

    device = _check_cuda(table_device, grad_scale)
    if grad_scale.dtype != torch.float32 or grad_scale.numel() != 1:
        raise ValueError("grad_scale must be one fp32 element")
    _lib.call(
        "pt_adamw_step_scaled",
        table_device.data_ptr(), table_device.size(0), int(total_blocks), float(lr), float(beta1),
        float(beta2), float(eps), float(weight_decay), float(step), grad_scale.data_ptr(),
        int(write_grad), _stream(device),
    )


def adamw_step_table(params: list[Tensor], steps: list[Tensor]) -> Tensor:
    """Host int64 [n] addresses of the fp32 device step of each parameter, in the row order
    of :func:`adamw_table` (which skips empty parameters)."""

    addrs = [s.data_ptr() for p, s in zip(params, steps) if p.numel() > 0]
    return torch.from_numpy(np.array(addrs, dtype=np.int64))


def adamw_step_device_step(
    table_device: Tensor,
    total_blocks: int,
    step_table_device: Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    grad_scale: Tensor | None = None,
    write_grad: bool = False,
    found_inf: Tensor | None = None,
    inv_scale: Tensor | None = None,
) -> None:
    """:func:`adamw_step` (or :func:`adamw_step_scaled` with ``grad_scale``) for a capturable
    optimizer: the step counts are fp32 device scalars, already advanced, whose addresses
    ``step_table_device`` lists in table row order.  With ``found_inf`` (the int32 flag of
    :func:`grad_stats`; needs ``grad_scale`` and ``inv_scale``) the update runs only when the
    flag is 0; when it is set the gradients are only multiplied by ``inv_scale``, decided on
    the device (advance the step counts by ``1 - found_inf``)."""

    device = _check_cuda(table_device, step_table_device)
    if step_table_device.dtype != torch.int64 or step_table_device.numel() != table_device.size(0):
        raise ValueError("the step table needs one int64 address per table row")
    for name, t, dtype in (("grad_scale", grad_scale, torch.float32), ("inv_scale", inv_scale, torch.float32),
                           ("found_inf", found_inf, torch.int32)):
        if t is not None:
            _check_cuda(t)
            if t.dtype != dtype or t.numel() != 1:
                raise ValueError(f"{name} must be one {dtype} element")
    if found_inf is None:
        _lib.call(
            "pt_adamw_step_device_step",
            table_device.data_ptr(), table_device.size(0), int(total_blocks), step_table_device.data_ptr(),
            float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), _ptr(grad_scale),
            int(write_grad), _stream(device),
        )
        return
    if grad_scale is None or inv_scale is None:
        raise ValueError("a guarded step needs grad_scale and inv_scale")
    _lib.call(
        "pt_adamw_step_device_step_guarded",
        table_device.data_ptr(), table_device.size(0), int(total_blocks), step_table_device.data_ptr(),
        float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), grad_scale.data_ptr(),
        int(write_grad), found_inf.data_ptr(), inv_scale.data_ptr(), _stream(device),
    )


def clip_grad_norm(table_device: Tensor, total_blocks: int, max_norm: float) -> tuple[Tensor, Tensor]:
    """(total_norm, clip_coef) fp32 device scalars over the gradients of a table built by
    :func:`adamw_table`: torch.nn.utils.clip_grad_norm_'s norm and clamped coefficient."""

    device = _check_cuda(table_device)
    out = torch.empty(2, dtype=torch.float32, device=device)
    ws_bytes = _lib.lib().pt_clip_grad_norm_workspace_bytes(int(total_blocks))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    _lib.call(
        "pt_clip_grad_norm",
        table_device.data_ptr(), table_device.size(0), int(total_blocks), float(max_norm),
        out.data_ptr(), out.data_ptr() + 4, ws.data_ptr(), ws_bytes, _stream(device),
    )
    return out[0], out[1:2]


CLIP_CLAMP = 0         # torch.nn.utils.clip_grad_norm_: g *= min(coef, 1)
CLIP_IF_BELOW_ONE = 1  # the ZeRO optimizer: g *= coef only when coef < 1


def grad_stats(
    table_device: Tensor,
    total_blocks: int,
    inv_scale: Tensor | None = None,
    max_norm: float | None = None,
    clip_mode: int = CLIP_CLAMP,
) -> tuple[Tensor, Tensor, Tensor]:
    """(total_norm, grad_scale, found_inf) device scalars over a table's gradients: the
    norm of g * inv_scale, inv_scale times the clip coefficient (1 without ``max_norm``),
    and whether any gradient is inf or NaN (int32)."""

    device = _check_cuda(table_device)
    if inv_scale is not None:
        _check_cuda(inv_scale)
        if inv_scale.dtype != torch.float32 or inv_scale.numel() != 1:
            raise ValueError("inv_scale must be one fp32 element")
    out = torch.empty(3, dtype=torch.float32, device=device)
    ws_bytes = _lib.lib().pt_grad_stats_workspace_bytes(int(total_blocks))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    _lib.call(
        "pt_grad_stats",
        table_device.data_ptr(), table_device.size(0), int(total_blocks), _ptr(inv_scale),
        -1.0 if max_norm is None else float(max_norm), int(clip_mode), out.data_ptr(),
        out.data_ptr() + 4, out.data_ptr() + 8, ws.data_ptr(), ws_bytes, _stream(device),
    )
    return out[0], out[1:2], out[2:3].view(torch.int32)


def grad_scale(table_device: Tensor, total_blocks: int, scale: Tensor) -> None:
    """g *= scale (fp32 device scalar) in place for every gradient of a table."""

    device = _check_cuda(table_device, scale)
    _lib.call("pt_grad_scale", table_device.data_ptr(), table_device.size(0), int(total_blocks),
              scale.data_ptr(), _stream(device))


# ------------------------------------------------------------------ utility


def copy_bytes(src: Tensor, dst: Tensor) -> None:
    """128-bit streaming device copy of src into dst (same byte size)."""

    device = _check_cuda(src, dst)
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes or not src.is_contiguous() or not dst.is_contiguous():
        raise ValueError("copy_bytes needs contiguous tensors of equal byte size")
    _lib.call("pt_copy", src.data_ptr(), dst.data_ptr(), nbytes, _stream(device))


# ------------------------------------------------------------------ torch.compile
#
# The launchers of the ops a compiled model contains (RMSNorm, the residual add + norm, SwiGLU,
# RoPE) as custom operators: torch.compile records a call as one opaque node (no graph break
# at the ctypes call) and propagates shapes through the fake implementations; the compiled
# graph calls the launcher eagerly.  Every output is a new tensor.  The cross-entropy and the
# optimizer step run outside picotron's compiled model (train_loop.py:136-168) and keep only
# their eager path.


@torch.library.custom_op("picotron_amd::rmsnorm_fwd", mutates_args=())
def _op_rmsnorm_fwd(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return rmsnorm_fwd(x, weight, eps)


@_op_rmsnorm_fwd.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape), x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.custom_op("picotron_amd::rmsnorm_bwd", mutates_args=())
def _op_rmsnorm_bwd(dy: Tensor, x: Tensor, weight: Tensor, rstd: Tensor) -> tuple[Tensor, Tensor]:
    return rmsnorm_bwd(dy, x, weight, rstd)


@_op_rmsnorm_bwd.register_fake
def _(dy, x, weight, rstd):
    return x.new_empty(x.shape), weight.new_empty((x.size(-1),))


@torch.library.custom_op("picotron_amd::residual_rmsnorm_fwd", mutates_args=())
def _op_residual_rmsnorm_fwd(
    x: Tensor, residual: Tensor, weight: Tensor, eps: float
) -> tuple[Tensor, Tensor, Tensor]:
    return residual_rmsnorm_fwd(x, residual, weight, eps)


@_op_residual_rmsnorm_fwd.register_fake
def _(x, residual, weight, eps):
    return x.new_empty(x.shape), x.new_empty(x.shape), x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.custom_op("picotron_amd::residual_rmsnorm_bwd", mutates_args=())
def _op_residual_rmsnorm_bwd(
    dy: Tensor, dh_in: Tensor | None, h: Tensor, weight: Tensor, rstd: Tensor
) -> tuple[Tensor, Tensor]:
    return residual_rmsnorm_bwd(dy, dh_in, h, weight, rstd)


@_op_residual_rmsnorm_bwd.register_fake
def _(dy, dh_in, h, weight, rstd):
    return h.new_empty(h.shape), weight.new_empty((h.size(-1),))


@torch.library.custom_op("picotron_amd::swiglu_fwd", mutates_args=())
def _op_swiglu_fwd(gate: Tensor, up: Tensor) -> Tensor:
    return swiglu_fwd(gate, up)


@_op_swiglu_fwd.register_fake
def _(gate, up):
    return gate.new_empty(gate.shape)


@torch.library.custom_op("picotron_amd::swiglu_bwd", mutates_args=())
def _op_swiglu_bwd(dout: Tensor, gate: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    return swiglu_bwd(dout, gate, up)


@_op_swiglu_bwd.register_fake
def _(dout, gate, up):
    return gate.new_empty(gate.shape), up.new_empty(up.shape)


@torch.library.custom_op("picotron_amd::rope", mutates_args=())
def _op_rope(x: Tensor, cos: Tensor, sin: Tensor, layout: str, inverse: bool) -> Tensor:
    return rope(x, cos, sin, layout=layout, inverse=inverse)[0]


@_op_rope.register_fake
def _(x, cos, sin, layout, inverse):
    return torch.empty_like(x)


@torch.library.custom_op("picotron_amd::rope_pair", mutates_args=())
def _op_rope_pair(
    x0: Tensor, x1: Tensor, cos: Tensor, sin: Tensor, layout: str, inverse: bool
) -> tuple[Tensor, Tensor]:
    y0, y1 = rope(x0, cos, sin, layout=layout, inverse=inverse, x1=x1)
    return y0, y1


@_op_rope_pair.register_fake
def _(x0, x1, cos, sin, layout, inverse):
    return torch.empty_like(x0), torch.empty_like(x1)
