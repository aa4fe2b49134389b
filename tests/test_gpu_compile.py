"""The fused modules under torch.compile: a block of RMSNorm, RoPE, the residual add + norm and
SwiGLU compiles into ONE graph (the launchers are custom operators, opaque to the compiler),
its compiled forward and backward launch the HIP kernels, and they match the eager modules.

A model wrapped in torch.compile reaches these ops through the same modules (reference src/picotron/models/picotron_decoder.py:20-46,
src/picotron/nn/feedforward.py:13-43), and picotron's `compile_model` option does so itself.
The main test uses the "aot_eager" backend: it traces forward and backward through
AOTAutograd and runs the graphs eagerly, so it needs no code generator; the last one uses the
default backend, as that option does.
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
