"""Tensors above 2^31 elements (HBM holds them easily: each is 4.3 GB in bf16).

Every offset past element 2^31 needs 64-bit index arithmetic, so each test puts data there
and checks against the oracle: the element-wise outputs on slices at the start, across the
2^31 boundary and at the end, and the whole-tensor reductions (RMSNorm dW, the mean
cross-entropy) over every row, computed in chunks.
"""

from __future__ import annotations

import gc

import pytest
import torch

from gpu_util import BF16, close_fp32
from oracle import adamw as o_adamw
from oracle import cross_entropy as o_ce
from oracle import rmsnorm as o_rms
from oracle import rope as o_rope
from oracle import swiglu as o_swiglu
from picotron_amd import ops

pytestmark = pytest.mark.gpu

TWO31 = 1 << 31


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _randn(shape, dtype, device, seed, scale=1.0):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=dtype).mul_(scale)


def _windows(n: int, width: int) -> list[slice]:
    """Slices at the start, across the 2^31 boundary and at the end of n elements."""

    return [slice(0, width), slice(TWO31 - width // 2, TWO31 + width // 2), slice(n - width, n)]


@pytest.mark.parametrize("extra", [4104, 4099])  # whole 16-byte vectors / an element-wise tail
def test_swiglu_past_2_31_elements(gpu, extra):
    n = TWO31 + extra
    g = _randn(n, torch.bfloat16, gpu, 1)
    u = _randn(n, torch.bfloat16, gpu, 2)
    y = ops.swiglu_fwd(g, u)
    dy = _randn(n, torch.bfloat16, gpu, 3)
    dg, du = ops.swiglu_bwd(dy, g, u)
    torch.cuda.synchronize()
    for w in _windows(n, 1 << 20):
        torch.testing.assert_close(y[w].double(), o_swiglu.forward(g[w], u[w]), **BF16)
        eg, eu = o_swiglu.backward(dy[w], g[w], u[w])
        torch.testing.assert_close(dg[w].double(), eg, **BF16)
        torch.testing.assert_close(du[w].double(), eu, **BF16)


# The write-through stores address a whole output through one buffer resource with 31-bit
# byte offsets; outputs up to 2^31 - 1 bytes take them, larger ones the nontemporal global
# stores.  These cases sit at that limit on both sides.
_WT_VECS = 0x7FFFFFFF // 16  # 16-byte vectors of the largest write-through SwiGLU output


@pytest.mark.parametrize("n", [_WT_VECS * 8, _WT_VECS * 8 + 3, (_WT_VECS + 1) * 8])
def test_swiglu_backward_at_the_write_through_limit(gpu, n):
    g = _randn(n, torch.bfloat16, gpu, 21)
    u = _randn(n, torch.bfloat16, gpu, 22)
    dy = _randn(n, torch.bfloat16, gpu, 23)
    dg, du = ops.swiglu_bwd(dy, g, u)
    torch.cuda.synchronize()
    for w in (slice(0, 1 << 20), slice(n // 2, n // 2 + (1 << 20)), slice(n - (1 << 20), n)):
        eg, eu = o_swiglu.backward(dy[w], g[w], u[w])
        torch.testing.assert_close(dg[w].double(), eg, **BF16)
        torch.testing.assert_close(du[w].double(), eu, **BF16)


@pytest.mark.parametrize("s", [4095, 4097])  # output 2^31 - 2^19 bytes / over 2^31 bytes
def test_rope_at_the_write_through_limit(gpu, s):
    b, h, d = 64, 32, 128
    cos, sin = o_rope.tables(s, d, 500_000.0, device=gpu)
    x = _randn((b, s, h, d), torch.bfloat16, gpu, 24).transpose(1, 2)  # (B,H,S,D) of (B,S,H,D)
    for layout in ("interleaved", "rotate_half"):
        y, _ = ops.rope(x, cos, sin, layout=layout)
        torch.cuda.synchronize()
        for bi in (0, b - 1):
            torch.testing.assert_close(y[bi].double(), o_rope.rotate(x[bi], cos, sin, layout), **BF16)
        del y


def test_rmsnorm_past_2_31_elements(gpu):
    cols = 4096
    rows = TWO31 // cols + 13  # the last 13 rows start past element 2^31
    eps = 1e-5
    x = _randn((rows, cols), torch.bfloat16, gpu, 4)
    w = (1.0 + 0.02 * _randn(cols, torch.float32, gpu, 5))  # fp32 weight: an fp32 dW
    y, rstd = ops.rmsnorm_fwd(x, w, eps)
    dy = _randn((rows, cols), torch.bfloat16, gpu, 6)
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    torch.cuda.synchronize()
    for rs in (slice(0, 512), slice(rows - 600, rows)):
        ey, er = o_rms.forward(x[rs], w, eps)
        torch.testing.assert_close(y[rs].double(), ey, **BF16)
        close_fp32(rstd[rs], er)
        edx, _ = o_rms.backward(dy[rs], x[rs], w, eps)
        torch.testing.assert_close(dx[rs].double(), edx, **BF16)
    # dW over every row, in fp64 chunks; the tolerance is relative to the summed magnitudes
    want = torch.zeros(cols, dtype=torch.float64, device=gpu)
    mag = torch.zeros(cols, dtype=torch.float64, device=gpu)
    for r0 in range(0, rows, 16384):
        xc = x[r0:r0 + 16384].double()
        terms = dy[r0:r0 + 16384].double() * xc * torch.rsqrt((xc * xc).mean(-1, keepdim=True) + eps)
        want += terms.sum(0)
        mag += terms.abs().sum(0)
        del xc, terms
    err = (dw.double() - want).abs()
    assert bool((err <= 1e-6 * mag).all()), f"max err/mag {float((err / mag).max())}"


@pytest.mark.parametrize("vocab,rows", [(128256, TWO31 // 128256 + 40), (50257, TWO31 // 50257 + 40)])
def test_cross_entropy_past_2_31_elements(gpu, vocab, rows):
    # 128256: register-resident rows; 50257 (rows not 16-byte aligned): the batched kernel
    logits = _randn((rows, vocab), torch.bfloat16, gpu, 7, 2.0)
    gen = torch.Generator(device=gpu).manual_seed(8)
    targets = torch.randint(0, vocab, (rows,), generator=gen, device=gpu)
    targets[torch.randperm(rows, generator=gen, device=gpu)[: rows // 20]] = -100
    targets[-1] = vocab - 1  # the last element of the tensor is a target
    check = [slice(0, 64), slice(rows - 64, rows)]
    before = [logits[rs].clone() for rs in check]
    # the loss over every row, in fp64 chunks, before the in-place gradient overwrites them
    total = torch.zeros((), dtype=torch.float64, device=gpu)
    for r0 in range(0, rows, 2048):
        lc = logits[r0:r0 + 2048].double()
        tc = targets[r0:r0 + 2048]
        keep = tc != -100
        lse = torch.logsumexp(lc, dim=-1)
        picked = lc.gather(1, tc.clamp(min=0).unsqueeze(1)).squeeze(1)
        total += torch.where(keep, lse - picked, torch.zeros_like(lse)).sum()
        del lc
    n_valid = int((targets != -100).sum())
    loss, _ = ops.cross_entropy(logits, targets, write_grad=True)
    torch.cuda.synchronize()
    want = float(total) / n_valid
    assert abs(float(loss) - want) <= 1e-4 * abs(want)
    for rs, lg in zip(check, before):
        # the oracle normalises by its own slice's valid count: rescale to the whole batch's
        tc = targets[rs]
        _, eg = o_ce.forward_backward(lg, tc)
        eg = eg * (int((tc != -100).sum()) / n_valid)
        torch.testing.assert_close(logits[rs].double(), eg, atol=2e-2 / n_valid, rtol=1.6e-2)


def test_rope_past_2_31_elements(gpu):
    b, s, h, d = 64, 8200, 32, 128  # 2.15e9 elements, 1.07e9 rotation pairs
    cos, sin = o_rope.tables(s, d, 500_000.0, device=gpu)
    x = _randn((b, s, h, d), torch.bfloat16, gpu, 9).transpose(1, 2)  # (B,H,S,D) of (B,S,H,D)
    for layout in ("interleaved", "rotate_half"):
        y, _ = ops.rope(x, cos, sin, layout=layout)
        torch.cuda.synchronize()
        for bi in (0, b - 1):
            torch.testing.assert_close(y[bi].double(), o_rope.rotate(x[bi], cos, sin, layout), **BF16)
        del y


def test_adamw_past_2_31_elements(gpu):
    n = TWO31 + 1000
    p = torch.nn.Parameter(_randn(n, torch.float32, gpu, 10, 0.02))
    p.grad = _randn(n, torch.float32, gpu, 11, 1e-3)
    opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    windows = _windows(n, 1 << 20)
    p0 = [p.detach()[w].clone() for w in windows]
    from picotron_amd.nn.triton_kernels import triton_adamw_step

    triton_adamw_step(opt)
    torch.cuda.synchronize()
    st = opt.state[p]
    for w, pw in zip(windows, p0):
        zero = torch.zeros_like(pw)
        ep, em, ev = o_adamw.step(pw, p.grad[w], zero, zero, t=1, lr=3e-4, beta1=0.9, beta2=0.95,
                                  eps=1e-8, weight_decay=0.1)
        close_fp32(p.detach()[w], ep)
        close_fp32(st["exp_avg"][w], em)
        close_fp32(st["exp_avg_sq"][w], ev)
