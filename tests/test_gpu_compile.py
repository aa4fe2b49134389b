"""The fused modules under torch.compile: a block of RMSNorm, RoPE, the residual add + norm and
SwiGLU compiles into ONE graph (the launchers are custom operators, opaque to the compiler),
its compiled forward and backward launch the HIP kernels, and they match the eager modules.

A model wrapped in torch.compile reaches these ops through the same modules (reference src/picotron/models/picotron_decoder.py:20-46,
src/picotron/nn/feedforward.py:13-43), and picotron's `compile_model` option does so itself.
Most tests use the "aot_eager" backend: it traces forward and backward through AOTAutograd
and runs the graphs eagerly, so it needs no code generator; one uses the default backend, as
that option does.
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn

from gpu_util import BF16, close_fp32, randn
from picotron_amd import _lib
from picotron_amd.nn import RMSNorm, RotaryEmbedding, SwiGLU

pytestmark = pytest.mark.gpu

HIDDEN, INTER, HEADS = 256, 512, 4


class _Block(nn.Module):
    def __init__(self, layout: str) -> None:
        super().__init__()
        self.norm1 = RMSNorm(HIDDEN, use_triton_rmsnorm=True)
        self.qk = nn.Linear(HIDDEN, 2 * HIDDEN, bias=False)
        self.rope = RotaryEmbedding(HIDDEN // HEADS, use_triton_rope=True, layout=layout)
        self.norm2 = RMSNorm(HIDDEN, use_triton_rmsnorm=True)
        self.mlp = SwiGLU(HIDDEN, INTER, use_triton_swiglu=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, s, _ = x.shape
        h = self.norm1(x)
        q, k = self.qk(h).view(b, s, 2, HEADS, HIDDEN // HEADS).permute(2, 0, 3, 1, 4).unbind(0)
        q, k = self.rope(q, k)
        mixed = h + (q * k).mean(dim=(1, 3)).unsqueeze(-1)
        r, y = self.norm2.add_and_norm(mixed, x)
        return r + self.mlp(y)


def _count_launches(monkeypatch) -> dict[str, int]:
    counts: dict[str, int] = {}
    real = _lib.call

    def counting(fn, *args):
        counts[fn] = counts.get(fn, 0) + 1
        return real(fn, *args)

    monkeypatch.setattr(_lib, "call", counting)
    return counts


def _run(model, x, dy, module=None):
    x = x.detach().requires_grad_(True)
    out = model(x)
    out.backward(dy)
    grads = {n: p.grad.detach().clone() for n, p in (module or model).named_parameters()}
    return out.detach(), x.grad.detach(), grads


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["interleaved", "rotate_half"])
def test_block_compiles_to_one_graph_and_matches_eager(gpu, monkeypatch, dtype, layout):
    print(f"compile block dtype {dtype} layout {layout}", flush=True)
    torch._dynamo.reset()
    torch.manual_seed(0)
    eager = _Block(layout).to(gpu, dtype)
    compiled_model = copy.deepcopy(eager)
    x = randn((2, 64, HIDDEN), dtype, gpu, 1)
    dy = randn((2, 64, HIDDEN), dtype, gpu, 2)

    explained = torch._dynamo.explain(copy.deepcopy(eager))(x)
    assert explained.graph_break_count == 0, [str(b.reason) for b in explained.break_reasons]
    assert explained.graph_count == 1

    torch._dynamo.reset()
    compiled = torch.compile(compiled_model, backend="aot_eager", fullgraph=True)
    counts = _count_launches(monkeypatch)
    out_c, dx_c, grads_c = _run(compiled, x, dy, compiled_model)
    torch.cuda.synchronize()
    # every fused op of the block ran as its HIP kernel inside the compiled graphs
    for fn, n in [("pt_rmsnorm_fwd", 1), ("pt_residual_rmsnorm_fwd", 1), ("pt_swiglu_fwd", 1),
                  ("pt_swiglu_bwd", 1), ("pt_residual_rmsnorm_bwd", 1), ("pt_rope", 2)]:
        assert counts.get(fn, 0) == n, (fn, counts)
    assert counts.get("pt_rmsnorm_bwd", 0) == 1, counts

    out_e, dx_e, grads_e = _run(eager, x, dy)
    check = close_fp32 if dtype == torch.float32 else (
        lambda a, e: torch.testing.assert_close(a.double(), e.double(), **BF16)
    )
    check(out_c, out_e)
    check(dx_c, dx_e)
    for name in grads_e:
        check(grads_c[name], grads_e[name])


def test_block_compiles_with_the_default_backend(gpu, monkeypatch):
    """picotron's own `compile_model` option calls torch.compile(model) with the default
    backend (reference src/picotron/training/train_loop.py:230-241): the fused ops stay calls
    into the library inside the generated code.  fp32, where the code generator's fused
    elementwise ops round as eager does up to the last bits."""

    print("compile block, default backend, fp32", flush=True)
    torch._dynamo.reset()
    torch.manual_seed(0)
    eager = _Block("rotate_half").to(gpu, torch.float32)
    compiled_model = copy.deepcopy(eager)
    x = randn((2, 64, HIDDEN), torch.float32, gpu, 3)
    dy = randn((2, 64, HIDDEN), torch.float32, gpu, 4)
    compiled = torch.compile(compiled_model, fullgraph=True)
    counts = _count_launches(monkeypatch)
    out_c, dx_c, grads_c = _run(compiled, x, dy, compiled_model)
    torch.cuda.synchronize()
    for fn, n in [("pt_rmsnorm_fwd", 1), ("pt_residual_rmsnorm_fwd", 1), ("pt_swiglu_fwd", 1),
                  ("pt_swiglu_bwd", 1), ("pt_residual_rmsnorm_bwd", 1), ("pt_rope", 2),
                  ("pt_rmsnorm_bwd", 1)]:
        assert counts.get(fn, 0) == n, (fn, counts)
    out_e, dx_e, grads_e = _run(eager, x, dy)
    close_fp32(out_c, out_e)
    close_fp32(dx_c, dx_e)
    for name in grads_e:
        close_fp32(grads_c[name], grads_e[name])


def test_fused_loss_inside_a_compiled_function(gpu):
    """The fused cross-entropy is not a custom op: inside a compiled function the compiler
    runs it eagerly (a graph break at its library calls) and the result is the eager one, with
    no fallback to F.cross_entropy."""

    import warnings

    from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback

    torch._dynamo.reset()
    torch.manual_seed(1)
    head = nn.Linear(64, 1000, bias=False).to(gpu)
    x = randn((2, 33, 64), torch.float32, gpu, 5)
    ids = torch.randint(0, 1000, (2, 33), generator=torch.Generator(device=gpu).manual_seed(6), device=gpu)
    loss_fn = CrossEntropyWithFallback(use_triton=True, inplace=True)

    def step(inp):
        return loss_fn(head(inp), ids, shift=True)

    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        loss_c = torch.compile(step, backend="aot_eager")(x)
        loss_c.backward()
        grad_c = head.weight.grad.clone()
        head.weight.grad = None
        loss_e = step(x)
        loss_e.backward()
    assert loss_c.item() == loss_e.item()
    assert torch.equal(grad_c, head.weight.grad)


def test_compiled_decoder_trains_like_eager(gpu, monkeypatch):
    """The reference's own compile check (tests/test_torch_compile.py:30-49: three training
    steps of a compiled model give the eager losses within rtol 1e-5, atol 1e-6) on a small
    decoder with every fused kernel on: the model compiled, the fused loss and the fused
    clip + AdamW step outside it, as the train loop has them (train_loop.py:136-168).  The
    compiled model's weights then load unchanged into the same decoder on the PyTorch
    fallbacks (tests/test_torch_compile.py:52-71)."""

    import warnings

    from test_gpu_decoder_step import VOCAB, Decoder, _models
    from picotron_amd.nn.triton_kernels import AdamWStepWithFallback, CrossEntropyWithFallback

    torch._dynamo.reset()
    _, eager = _models(gpu)
    compiled_model = copy.deepcopy(eager)
    compiled = torch.compile(compiled_model, backend="aot_eager")
    batches = [torch.randint(0, VOCAB, (2, 65), generator=torch.Generator().manual_seed(40 + i)).to(gpu)
               for i in range(3)]

    def train(model, params):
        optimizer = torch.optim.AdamW(params, lr=2e-3, betas=(0.9, 0.95), weight_decay=0.1)
        loss_fn = CrossEntropyWithFallback(use_triton=True, inplace=True)
        stepper = AdamWStepWithFallback(use_triton=True)
        losses = []
        for ids in batches:
            optimizer.zero_grad(set_to_none=True)
            loss = loss_fn(model(ids), ids, shift=True)
            loss.backward()
            stepper.step(optimizer, max_grad_norm=1.0)
            losses.append(loss.item())
        return losses

    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)  # a fallback would warn
        eager_losses = train(eager, list(eager.parameters()))
        counts = _count_launches(monkeypatch)
        compiled_losses = train(compiled, list(compiled_model.parameters()))
    # per step: 2 blocks' input norms + the final norm, 2 residual norms, 2 SwiGLUs, 2 RoPE
    # launches per block forward and backward, the shifted loss, the clip and the step
    for fn, n in [("pt_rmsnorm_fwd", 3), ("pt_rmsnorm_bwd", 3), ("pt_residual_rmsnorm_fwd", 2),
                  ("pt_residual_rmsnorm_bwd", 2), ("pt_swiglu_fwd", 2), ("pt_swiglu_bwd", 2),
                  ("pt_rope", 4), ("pt_cross_entropy_shifted", 1), ("pt_clip_grad_norm", 1),
                  ("pt_adamw_step_scaled", 1)]:
        assert counts.get(fn, 0) == 3 * n, (fn, counts)
    print(f"eager losses {eager_losses} compiled {compiled_losses}", flush=True)
    torch.testing.assert_close(torch.tensor(compiled_losses), torch.tensor(eager_losses),
                               rtol=1e-5, atol=1e-6)
    assert compiled_losses[-1] < compiled_losses[0]

    portable = Decoder(fused=False).to(gpu)
    portable.load_state_dict(compiled_model.state_dict())
    for name, value in compiled_model.state_dict().items():
        assert torch.equal(portable.state_dict()[name], value), name
