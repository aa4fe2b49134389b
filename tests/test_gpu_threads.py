"""Concurrent use of the library: several host threads, each on its own stream (default
priority), drive the fused kernels on their own tensors at once; every result equals the same
call made alone (the kernels are deterministic, so bit for bit).  The C ABI keeps no state
between calls besides per-device properties initialised once, and the autograd engine calls
the backwards from its own device thread, so calls from several threads must not interfere."""

from __future__ import annotations

import threading

import pytest
import torch

from gpu_util import randn
from oracle import rope as o_rope
from picotron_amd import ops
from picotron_amd.nn.triton_kernels import triton_adamw_step

pytestmark = pytest.mark.gpu

THREADS, ITERS = 4, 6


def _inputs(gpu, t):
    seed = 900 + 20 * t
    d = dict(
        x=randn((1024 + 64 * t, 4096), torch.bfloat16, gpu, seed),
        w=randn((4096,), torch.bfloat16, gpu, seed + 1, 0.02, 1.0),
        dy=randn((1024 + 64 * t, 4096), torch.bfloat16, gpu, seed + 2),
        g=randn((2_000_000 + 1000 * t,), torch.bfloat16, gpu, seed + 3),
        u=randn((2_000_000 + 1000 * t,), torch.bfloat16, gpu, seed + 4),
        logits=randn((64 + t, 32000), torch.bfloat16, gpu, seed + 5, 2.0),
        q=randn((2, 128, 8, 64), torch.bfloat16, gpu, seed + 6).transpose(1, 2),
        k=randn((2, 128, 2, 64), torch.bfloat16, gpu, seed + 7).transpose(1, 2),
    )
    d["targets"] = torch.randint(0, 32000, (64 + t,), generator=torch.Generator(device=gpu).manual_seed(seed + 8),
                                 device=gpu)
    d["cos"], d["sin"] = o_rope.tables(128, 64, 500_000.0, device=gpu)
    return d


def _work(d):
    y, rstd = ops.rmsnorm_fwd(d["x"], d["w"], 1e-5)
    dx, dw = ops.rmsnorm_bwd(d["dy"], d["x"], d["w"], rstd)
    out = ops.swiglu_fwd(d["g"], d["u"])
    dg, du = ops.swiglu_bwd(out, d["g"], d["u"])
    buf = d["logits"].clone()
    loss, _ = ops.cross_entropy(buf, d["targets"], write_grad=True)
    yq, yk = ops.rope(d["q"], d["cos"], d["sin"], layout="rotate_half", x1=d["k"])
    return [y, rstd, dx, dw, out, dg, du, buf, loss, yq, yk]


def _adamw_state(gpu, t):
    params = [torch.nn.Parameter(randn((n,), torch.float32, gpu, 950 + 10 * t + i, 0.02))
              for i, n in enumerate((300_000, 4096, 1_000_001))]
    for i, p in enumerate(params):
        p.grad = randn(p.shape, torch.float32, gpu, 990 + 10 * t + i, 1e-3)
    return params, torch.optim.AdamW(params, lr=1e-3, weight_decay=0.1)


def test_threads_on_their_own_streams_match_single_calls(gpu):
    inputs = [_inputs(gpu, t) for t in range(THREADS)]
    expected = [_work(d) for d in inputs]
    serial = []
    for t in range(THREADS):
        params, opt = _adamw_state(gpu, t)
        for _ in range(ITERS):
            triton_adamw_step(opt)
        serial.append([p.detach().clone() for p in params])
    torch.cuda.synchronize()

    results: list = [None] * THREADS
    errors: list = []
    start = threading.Barrier(THREADS)
    states = [_adamw_state(gpu, t) for t in range(THREADS)]
    torch.cuda.synchronize()

    def run(t):
        try:
            stream = torch.cuda.Stream(device=gpu)
            stream.wait_stream(torch.cuda.default_stream(gpu))
            start.wait()
            with torch.cuda.stream(stream):
                outs = None
                for _ in range(ITERS):
                    outs = _work(inputs[t])
                    triton_adamw_step(states[t][1])
            stream.synchronize()
            results[t] = outs
        except Exception as error:  # reported by the main thread
            errors.append((t, error))

    threads = [threading.Thread(target=run, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(THREADS):
        print(f"thread {t}: comparing {len(expected[t])} outputs and the optimizer", flush=True)
        for i, (a, e) in enumerate(zip(results[t], expected[t])):
            assert torch.equal(a, e), (t, i)
        for p, ref in zip(states[t][0], serial[t]):
            assert torch.equal(p.detach(), ref), t
