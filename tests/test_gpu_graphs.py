"""HIP graph capture of the fused kernels.

Each fused call (forward and backward through autograd) is captured once with
``torch.cuda.graph`` and replayed several times. Between replays, ordinary eager work writes
new inputs into the captured buffers and the device is synchronised. Every replay must equal
the eager call on the same inputs bit for bit: the kernels are deterministic, so a replay that
read stale workspace, a value frozen at capture time or a buffer freed since would show up as
a mismatch. None of these paths issues a memset, a host read or an allocation of its own
inside the capture (workspaces come from torch's allocator, which serves a capture from the
graph's private pool).
"""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

from picotron_amd.nn.triton_kernels import (
    triton_apply_rotary_embedding_pair,
    triton_cross_entropy,
    triton_residual_rms_norm,
    triton_rms_norm,
    triton_swiglu,
    triton_zero_clip_grad_norm_,
)
from oracle import rope as o_rope
from picotron_amd.nn.triton_kernels.adamw import TritonAdamWUnavailable

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _capture(fn, inputs):
    """Runs ``fn(*inputs)`` twice on a side stream (the warm-up that builds any cached
    tables), then captures it; returns the graph and the captured call's outputs."""

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn(*inputs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = fn(*inputs)
    return graph, outputs


def _check_replays(fn, inputs, fill):
    """Captures ``fn`` on ``inputs``; for each replay, ``fill(inputs, i)`` writes new values
    in place (eager), the graph replays, and its outputs must equal an eager call of ``fn``
    on clones of the same inputs."""

    fill(inputs, 0)
    graph, outputs = _capture(fn, inputs)
    for i in range(1, REPLAYS + 1):
        fill(inputs, i)
        torch.cuda.synchronize()
        clones = [t.detach().clone().requires_grad_(t.requires_grad) for t in inputs]
        graph.replay()
        torch.cuda.synchronize()
        expected = fn(*clones)
        torch.cuda.synchronize()
        assert len(outputs) == len(expected)
        for k, (got, want) in enumerate(zip(outputs, expected)):
            assert got.dtype == want.dtype and got.shape == want.shape, (i, k)
            assert torch.equal(got, want), f"replay {i}, output {k}: max diff {(got.float() - want.float()).abs().max()}"


def _randn_(t: torch.Tensor, seed: int, scale: float = 1.0, shift: float = 0.0) -> None:
    g = torch.Generator(device=t.device).manual_seed(seed)
    with torch.no_grad():
        t.copy_(torch.randn(t.shape, generator=g, device=t.device, dtype=torch.float32) * scale + shift)


def _leaf(shape, dtype, gpu, requires_grad=True):
    return torch.empty(shape, dtype=dtype, device=gpu).requires_grad_(requires_grad)


@pytest.mark.parametrize("dtype,rows,cols", [(torch.bfloat16, 1000, 4096), (torch.float32, 77, 1000)])
def test_rmsnorm_forward_and_backward_replay(gpu, dtype, rows, cols):
    def fn(x, w, dy):
        y = triton_rms_norm(x, w, 1e-5)
        dx, dw = torch.autograd.grad(y, (x, w), dy)
        return y.detach(), dx, dw

    def fill(t, i):
        _randn_(t[0], 10 * i + 1)
        _randn_(t[1], 10 * i + 2, 0.1, 1.0)
        _randn_(t[2], 10 * i + 3)

    inputs = [_leaf((rows, cols), dtype, gpu), _leaf((cols,), dtype, gpu), _leaf((rows, cols), dtype, gpu, False)]
    _check_replays(fn, inputs, fill)


def test_residual_rmsnorm_replay(gpu):
    rows, cols = 512, 2048

    def fn(x, r, w, dh, dy):
        h, y = triton_residual_rms_norm(x, r, w, 1e-6)
        dx, dr, dw = torch.autograd.grad((h, y), (x, r, w), (dh, dy))
        return h.detach(), y.detach(), dx, dr, dw

    def fill(t, i):
        for k, s in enumerate(t):
            _randn_(s, 10 * i + k, 0.1 if k == 2 else 1.0, 1.0 if k == 2 else 0.0)

    f32 = torch.float32
    inputs = [_leaf((rows, cols), f32, gpu), _leaf((rows, cols), f32, gpu), _leaf((cols,), f32, gpu),
              _leaf((rows, cols), f32, gpu, False), _leaf((rows, cols), f32, gpu, False)]
    _check_replays(fn, inputs, fill)


def test_swiglu_replay(gpu):
    shape = (3, 333, 1000)

    def fn(g, u, dy):
        y = triton_swiglu(g, u)
        dg, du = torch.autograd.grad(y, (g, u), dy)
        return y.detach(), dg, du

    def fill(t, i):
        for k, s in enumerate(t):
            _randn_(s, 10 * i + k)

    b = torch.bfloat16
    inputs = [_leaf(shape, b, gpu), _leaf(shape, b, gpu), _leaf(shape, b, gpu, False)]
    _check_replays(fn, inputs, fill)


@pytest.mark.parametrize("layout", ["interleaved", "rotate_half"])
def test_rope_pair_replay(gpu, layout):
    batch, seq, hq, hk, dim = 2, 128, 8, 2, 128
    cos, sin = o_rope.tables(seq, dim, 500_000.0, device=gpu)

    def fn(q, k, dq_out, dk_out):
        # (B, H, S, D) views of (B, S, H, D) memory, as attention passes them
        qv, kv = q.transpose(1, 2), k.transpose(1, 2)
        out_q, out_k = triton_apply_rotary_embedding_pair(qv, kv, cos, sin, layout=layout)
        dq, dk = torch.autograd.grad((out_q, out_k), (q, k), (dq_out.transpose(1, 2), dk_out.transpose(1, 2)))
        return out_q.detach().contiguous(), out_k.detach().contiguous(), dq, dk

    def fill(t, i):
        for k, s in enumerate(t):
            _randn_(s, 10 * i + k)

    b = torch.bfloat16
    inputs = [_leaf((batch, seq, hq, dim), b, gpu), _leaf((batch, seq, hk, dim), b, gpu),
              _leaf((batch, seq, hq, dim), b, gpu, False), _leaf((batch, seq, hk, dim), b, gpu, False)]
    _check_replays(fn, inputs, fill)


@pytest.mark.parametrize("shift", [False, True])
def test_cross_entropy_replay(gpu, shift):
    vocab = 50257  # unaligned rows take the batched kernel; see the aligned case below
    rows = 96

    def fn(logits, targets, grad_scale):
        loss = triton_cross_entropy(logits, targets, shift=shift, inplace=False)
        (grad,) = torch.autograd.grad(loss, (logits,), grad_scale)
        return loss.detach(), grad

    def fill(t, i):
        _randn_(t[0], 10 * i + 1, 2.0)
        g = torch.Generator(device=gpu).manual_seed(10 * i + 2)
        with torch.no_grad():
            t[1].copy_(torch.randint(0, vocab, t[1].shape, generator=g, device=gpu))
            t[1].view(-1)[torch.randperm(t[1].numel(), generator=g, device=gpu)[: 5 + i]] = -100
            t[2].fill_(1.0 if i % 2 else 0.5)  # the gradient scale changes between replays too

    shape = (2, rows // 2, vocab) if shift else (rows, vocab)
    tshape = (2, rows // 2) if shift else (rows,)
    inputs = [_leaf(shape, torch.bfloat16, gpu), torch.empty(tshape, dtype=torch.int64, device=gpu),
              torch.empty((), dtype=torch.float32, device=gpu)]
    _check_replays(fn, inputs, fill)


def test_cross_entropy_register_rows_replay(gpu):
    vocab, rows = 128256, 64

    def fn(logits, targets):
        loss = triton_cross_entropy(logits, targets, inplace=False)
        (grad,) = torch.autograd.grad(loss, (logits,))
        return loss.detach(), grad

    def fill(t, i):
        _randn_(t[0], 10 * i + 1, 2.0)
        g = torch.Generator(device=gpu).manual_seed(10 * i + 2)
        with torch.no_grad():
            t[1].copy_(torch.randint(0, vocab, t[1].shape, generator=g, device=gpu))
            t[1][i] = -100

    inputs = [_leaf((rows, vocab), torch.bfloat16, gpu), torch.empty((rows,), dtype=torch.int64, device=gpu)]
    _check_replays(fn, inputs, fill)


def test_zero_clip_grad_norm_replay(gpu):
    shapes = [(1000, 37), (4096,), (3, 5, 7), (1,)]
    params = [torch.zeros(s, device=gpu, requires_grad=True) for s in shapes]
    for p in params:
        p.grad = torch.empty_like(p)

    def fn(*grads):
        if grads[0] is params[0].grad:
            owners = params
        else:  # the eager check: fresh parameters holding the cloned gradients
            owners = [torch.zeros_like(p, requires_grad=True) for p in params]
            for p, g in zip(owners, grads):
                p.grad = g
        total = triton_zero_clip_grad_norm_(owners, 1.0)
        return [total] + [p.grad for p in owners]

    def fill(t, i):
        # replays alternate between a norm above max_norm (clipped) and below (kept)
        for k, s in enumerate(t):
            _randn_(s, 10 * i + k, 0.05 if i % 2 else 1e-4)

    _check_replays(fn, [p.grad for p in params], fill)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_clip_table_must_be_built_before_capture(gpu):
    p = torch.zeros(123, device=gpu, requires_grad=True)
    p.grad = torch.ones_like(p)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with pytest.raises(TritonAdamWUnavailable, match="before capturing"):
            with torch.cuda.graph(graph, stream=side):
                triton_zero_clip_grad_norm_([p], 1.0)
    torch.cuda.synchronize()


_FIRST_LAUNCH_IN_CAPTURE = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    import torch
    from picotron_amd import ops
    dev = torch.device("cuda:0")
    n = 1 << 22
    g, u, dy = (torch.randn(n, device=dev).bfloat16() for _ in range(3))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            dg, du = ops.swiglu_bwd(dy, g, u)
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        g.copy_(torch.randn(n, device=dev).bfloat16())
        graph.replay()
        torch.cuda.synchronize()
        eg, eu = ops.swiglu_bwd(dy, g, u)
        torch.cuda.synchronize()
        assert torch.equal(dg, eg) and torch.equal(du, eu), i
    print("ok")
""")


def test_first_launch_inside_a_capture(gpu):
    """A fresh process whose first SwiGLU backward launch is captured: that launch raises the
    kernel's dynamic LDS limit (its occupancy limit needs more than 64 KB) during the capture,
    and every replay must still equal the eager call."""

    root = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-c", _FIRST_LAUNCH_IN_CAPTURE.format(root=root)],
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0 and proc.stdout.strip().endswith("ok"), proc.stdout + proc.stderr
