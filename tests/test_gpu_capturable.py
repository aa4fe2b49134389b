"""The fused AdamW step for ``torch.optim.AdamW(..., capturable=True)``, whose step counts
live on the device, and a whole training step captured in one HIP graph.

The reference's fallback for such an optimizer is torch's own capturable step
(``optimizer.step()``, reference src/picotron/nn/triton_kernels/adamw.py:47); the fused step
must match it within the fp32 tolerance and leave the same state (device fp32 steps).
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from gpu_util import close_fp32, randn
from picotron_amd.nn import RMSNorm
from picotron_amd.nn.triton_kernels import (
    CrossEntropyWithFallback,
    triton_adamw_step,
    triton_clip_grad_norm_and_step,
    triton_swiglu,
)

pytestmark = pytest.mark.gpu

HP = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


@pytest.mark.parametrize("foreach", [False, True])
def test_capturable_step_matches_torch_capturable_adamw(gpu, foreach):
    shapes = [(1000, 37), (4096,), (3, 5, 7), (0,), (1,), (257,)]
    fused = [nn.Parameter(randn(s, torch.float32, gpu, i, 0.02)) for i, s in enumerate(shapes)]
    ref = [nn.Parameter(p.detach().clone()) for p in fused]
    opt_f = torch.optim.AdamW(fused, capturable=True, **HP)
    opt_r = torch.optim.AdamW(ref, capturable=True, foreach=foreach, **HP)
    for step in range(3):
        for i, (a, b) in enumerate(zip(fused, ref)):
            g = randn(a.shape, torch.float32, gpu, 100 * step + i, 1e-3)
            a.grad, b.grad = g, g.clone()
        triton_adamw_step(opt_f)
        opt_r.step()
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        sf, sr = opt_f.state[a], opt_r.state[b]
        close_fp32(sf["exp_avg"], sr["exp_avg"])
        close_fp32(sf["exp_avg_sq"], sr["exp_avg_sq"])
        assert sf["step"].device == a.device and sf["step"].dtype == torch.float32
        assert float(sf["step"]) == float(sr["step"]) == 3.0


def test_capturable_clip_and_step_match_torch(gpu):
    shapes = [(513, 64), (64,), (7,)]
    fused = [nn.Parameter(randn(s, torch.float32, gpu, 10 + i, 0.02)) for i, s in enumerate(shapes)]
    ref = [nn.Parameter(p.detach().clone()) for p in fused]
    opt_f = torch.optim.AdamW(fused, capturable=True, **HP)
    opt_r = torch.optim.AdamW(ref, capturable=True, foreach=False, **HP)
    for step in range(2):
        for i, (a, b) in enumerate(zip(fused, ref)):
            g = randn(a.shape, torch.float32, gpu, 50 * step + i, 0.1)  # norm well above 1
            a.grad, b.grad = g, g.clone()
        norm_f = triton_clip_grad_norm_and_step(opt_f, 1.0)
        norm_r = torch.nn.utils.clip_grad_norm_(ref, 1.0)
        opt_r.step()
        close_fp32(norm_f, norm_r)
    for a, b in zip(fused, ref):
        close_fp32(a.detach(), b.detach())
        close_fp32(a.grad, b.grad)  # left clipped, as clip_grad_norm_ leaves them


V, B, S = 512, 2, 33


def _model(gpu) -> nn.ModuleList:
    torch.manual_seed(3)
    norms = nn.ModuleList([RMSNorm(V, use_triton_rmsnorm=True), RMSNorm(V, use_triton_rmsnorm=True)]).to(gpu)
    with torch.no_grad():
        for n in norms:
            n.weight.add_(0.05 * torch.randn(V, device=gpu))
    for p in norms.parameters():
        p.grad = torch.zeros_like(p)  # gradients accumulate in place: stable addresses
    return norms


def _train_step(model, opt, loss_fn, x, ids):
    for p in model.parameters():
        p.grad.zero_()
    logits = triton_swiglu(model[0](x), model[1](0.5 * x + 1.0))
    loss = loss_fn(logits, ids, shift=True)
    loss.backward()
    triton_clip_grad_norm_and_step(opt, 1.0)
    return loss.detach()


def _inputs(gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn((B, S, V), generator=g, device=gpu) * 2.0
    ids = torch.randint(0, V, (B, S), generator=g, device=gpu)
    ids[0, 5] = -100
    return x, ids


def test_whole_training_step_replays_in_a_graph(gpu):
    """Forward, backward, clip and capturable AdamW step of fused modules in one graph;
    every replay equals the same step run eagerly, bit for bit (all kernels deterministic)."""

    graph_model, eager_model = _model(gpu), _model(gpu)
    graph_opt = torch.optim.AdamW(graph_model.parameters(), capturable=True, **HP)
    eager_opt = torch.optim.AdamW(eager_model.parameters(), capturable=True, **HP)
    graph_loss_fn = CrossEntropyWithFallback(use_triton=True, inplace=True)
    eager_loss_fn = CrossEntropyWithFallback(use_triton=True, inplace=True)
    x_static, ids_static = _inputs(gpu, 0)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up: state creation and the cached tables
            _train_step(graph_model, graph_opt, graph_loss_fn, x_static, ids_static)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(2):
        _train_step(eager_model, eager_opt, eager_loss_fn, x_static, ids_static)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = _train_step(graph_model, graph_opt, graph_loss_fn, x_static, ids_static)

    for i in range(1, 5):
        x, ids = _inputs(gpu, i)
        x_static.copy_(x)
        ids_static.copy_(ids)
        graph.replay()
        torch.cuda.synchronize()
        eager_loss = _train_step(eager_model, eager_opt, eager_loss_fn, x, ids)
        torch.cuda.synchronize()
        assert torch.equal(static_loss, eager_loss), i
        for (name, a), b in zip(graph_model.named_parameters(), eager_model.parameters()):
            assert torch.equal(a.detach(), b.detach()), (i, name)
            assert torch.equal(a.grad, b.grad), (i, name)
            for key in ("step", "exp_avg", "exp_avg_sq"):
                assert torch.equal(graph_opt.state[a][key], eager_opt.state[b][key]), (i, name, key)
        assert float(graph_opt.state[next(graph_model.parameters())]["step"]) == 2.0 + i
