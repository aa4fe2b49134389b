"""Seeded random shapes, dtypes and layouts for every kernel family against the oracle: row
counts and hidden sizes off the tuned grid, odd vocabularies, strided and offset views, long
parameter lists.  Each case prints its parameters first, so a failure names it.  The checks
are the per-family ones of the other parity tests (same tolerances).  PT_RANDOM_CASES sets the
number of cases per family (default 100; some families run half as many)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import test_gpu_cross_entropy as t_ce
import test_gpu_residual_rmsnorm as t_res
import test_gpu_rmsnorm as t_rms
import test_gpu_swiglu as t_swiglu
from gpu_util import close, close_fp32, randn
from oracle import rope as o_rope
from picotron_amd import ops
from picotron_amd.nn.triton_kernels import triton_adamw_step, triton_clip_grad_norm_and_step

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
CASES = int(os.environ.get("PT_RANDOM_CASES", "100"))


def _rng(family: str, case: int) -> np.random.Generator:
    return np.random.default_rng([sum(map(ord, family)), case])


def _log_uniform(rng, lo: int, hi: int) -> int:
    return int(round(float(np.exp(rng.uniform(np.log(lo), np.log(hi))))))


@pytest.mark.parametrize("case", range(CASES))
def test_rmsnorm_random(gpu, case):
    rng = _rng("rmsnorm", case)
    rows = _log_uniform(rng, 1, 3000)
    cols = _log_uniform(rng, 1, 20000)
    dtype = DTYPES[rng.integers(3)]
    wdtype = DTYPES[rng.integers(3)]
    pad = int(rng.integers(0, 3)) * int(rng.integers(1, 40))  # row stride cols + pad
    offset = int(rng.integers(0, 2)) * int(rng.integers(1, 9))  # element offset of the rows
    print(f"rmsnorm case {case}: rows {rows} cols {cols} {dtype} weight {wdtype} pad {pad} offset {offset}",
          flush=True)
    seed = 1000 + case
    big = randn((rows, offset + cols + pad), dtype, gpu, seed)
    x = big[:, offset:offset + cols]
    w = randn((cols,), wdtype, gpu, seed + 1, 0.02, 1.0)
    dy = randn((rows, cols), dtype, gpu, seed + 2)
    t_rms._check(x, w, 1e-5, dy, dtype)


@pytest.mark.parametrize("case", range(CASES // 2))
def test_residual_rmsnorm_random(gpu, case):
    rng = _rng("residual", case)
    rows = _log_uniform(rng, 1, 2000)
    cols = _log_uniform(rng, 2, 12000)
    dtype = DTYPES[rng.integers(3)]
    wdtype = DTYPES[rng.integers(3)]
    print(f"residual rmsnorm case {case}: rows {rows} cols {cols} {dtype} weight {wdtype}", flush=True)
    t_res._check(*t_res._case(gpu, (rows, cols), dtype, wdtype, 2000 + 5 * case), 1e-6, dtype)


@pytest.mark.parametrize("case", range(CASES))
def test_swiglu_random(gpu, case):
    rng = _rng("swiglu", case)
    n = _log_uniform(rng, 1, 3_000_000)
    dtype = DTYPES[rng.integers(3)]
    offsets = [int(rng.integers(0, 2)) * int(rng.integers(1, 8)) for _ in range(3)]
    print(f"swiglu case {case}: n {n} {dtype} offsets {offsets}", flush=True)
    seed = 3000 + 3 * case
    g = randn((n + offsets[0],), dtype, gpu, seed, 2.0)[offsets[0]:]
    u = randn((n + offsets[1],), dtype, gpu, seed + 1)[offsets[1]:]
    dy = randn((n + offsets[2],), dtype, gpu, seed + 2)[offsets[2]:]
    t_swiglu._check(g, u, dy, dtype)


@pytest.mark.parametrize("case", range(CASES))
def test_rope_random(gpu, case):
    rng = _rng("rope", case)
    b = int(rng.integers(1, 4))
    s = _log_uniform(rng, 1, 600)
    hk = int(rng.integers(1, 5))
    hq = hk * int(rng.integers(1, 5))
    d = 2 * _log_uniform(rng, 1, 128)
    layout = ["interleaved", "rotate_half"][rng.integers(2)]
    dtype = DTYPES[rng.integers(3)]
    extra = int(rng.integers(0, 3))  # table rows beyond the sequence
    bshd = bool(rng.integers(4))  # mostly attention's view, sometimes contiguous (B, H, S, D)
    print(f"rope case {case}: b {b} s {s} hq {hq} hk {hk} d {d} {layout} {dtype} "
          f"{'(B,S,H,D) memory' if bshd else 'contiguous'}", flush=True)
    seed = 4000 + 2 * case
    cos, sin = o_rope.tables(s + extra, d, 500_000.0, device=gpu)
    if bshd:
        # (B, H, S, D) views of (B, S, H, D) memory, as attention produces them
        q = randn((b, s, hq, d), dtype, gpu, seed).transpose(1, 2)
        k = randn((b, s, hk, d), dtype, gpu, seed + 1).transpose(1, 2)
    else:
        q = randn((b, hq, s, d), dtype, gpu, seed)
        k = randn((b, hk, s, d), dtype, gpu, seed + 1)
    yq, yk = ops.rope(q, cos, sin, layout=layout, x1=k)
    close(yq, o_rope.rotate(q, cos, sin, layout), dtype)
    close(yk, o_rope.rotate(k, cos, sin, layout), dtype)
    gq, gk = ops.rope(yq, cos, sin, layout=layout, inverse=True, x1=yk)
    close(gq, o_rope.rotate(yq, cos, sin, layout, inverse=True), dtype)
    close(gk, o_rope.rotate(yk, cos, sin, layout, inverse=True), dtype)


@pytest.mark.parametrize("case", range(CASES))
def test_cross_entropy_random(gpu, case):
    rng = _rng("ce", case)
    rows = _log_uniform(rng, 1, 700)
    vocab = _log_uniform(rng, 1, 200_000)
    dtype = DTYPES[rng.integers(3)]
    print(f"cross-entropy case {case}: rows {rows} vocab {vocab} {dtype}", flush=True)
    seed = 5000 + case
    logits = randn((rows, vocab), dtype, gpu, seed, 2.0)
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    ignored = torch.rand(rows, generator=g, device=gpu) < 0.1
    targets[ignored] = -100
    if not bool((targets != -100).any()):
        targets[0] = 0
    t_ce._check(logits, targets, dtype)


@pytest.mark.parametrize("case", range(CASES // 2))
def test_cross_entropy_train_loop_view_random(gpu, case):
    """The train loop's own call, F.cross_entropy(logits[:, :-1, :].transpose(1, 2),
    input_ids[:, 1:]) (reference train_loop.py:141-144): (B, V, S - 1) views whose class
    dimension is contiguous and whose rows are V apart; the gradient lands in the view and
    the last position of the buffer is left alone."""

    rng = _rng("ce_view", case)
    b = int(rng.integers(1, 4))
    s = _log_uniform(rng, 2, 300)
    v = _log_uniform(rng, 1, 150_000)
    dtype = DTYPES[rng.integers(3)]
    print(f"train-loop view cross-entropy case {case}: b {b} s {s} v {v} {dtype}", flush=True)
    seed = 8000 + case
    base = randn((b, s, v), dtype, gpu, seed, 2.0)
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    ids = torch.randint(0, v, (b, s), generator=g, device=gpu)
    ids[torch.rand((b, s), generator=g, device=gpu) < 0.1] = -100
    targets = ids[:, 1:]
    if not bool((targets != -100).any()):
        ids[0, 1] = 0
    view = base[:, :-1, :].transpose(1, 2)
    ref_loss, ref_grad = t_ce.o_ce.forward_backward(view, targets)
    n_valid = int((targets != -100).sum())
    loss, _ = ops.cross_entropy(view, targets)
    assert abs(loss.item() - ref_loss.item()) <= t_ce.LOSS_RTOL * abs(ref_loss.item())
    buf = base.clone()
    bview = buf[:, :-1, :].transpose(1, 2)
    loss2, ws = ops.cross_entropy(bview, targets, write_grad=True)
    assert abs(loss2.item() - ref_loss.item()) <= t_ce.LOSS_RTOL * abs(ref_loss.item())
    assert ops.cross_entropy_status(ws) == 0
    if dtype == torch.float16:
        # the backward writes the fp16 gradient at a GradScaler-sized scale (as in _check)
        scale = t_ce._fp16_scale_for(n_valid)
        ops.cross_entropy_scale_grad(bview, targets, torch.full((), scale, device=gpu), workspace=ws)
        t_ce._fp16_grad_close(bview, ref_grad, scale, n_valid)
    else:
        t_ce._grad_close(bview, ref_grad, n_valid, dtype)
    assert torch.equal(buf[:, -1, :], base[:, -1, :])


@pytest.mark.parametrize("case", range(CASES // 2))
def test_shifted_cross_entropy_random(gpu, case):
    rng = _rng("ce_shift", case)
    b = int(rng.integers(1, 4))
    s = _log_uniform(rng, 2, 300)
    v = _log_uniform(rng, 2, 150_000)
    dtype = DTYPES[rng.integers(3)]
    out_of_place = bool(rng.integers(2))
    print(f"shifted cross-entropy case {case}: b {b} s {s} v {v} {dtype} "
          f"{'out of place' if out_of_place else 'in place'}", flush=True)
    logits, ids = t_ce._shifted_case(gpu, b, s, v, dtype, 6000 + case)
    if not bool((ids[:, 1:] != -100).any()):
        ids[0, 1] = 0
    ref_loss, ref_grad = t_ce.o_ce.shifted_forward_backward(logits, ids)
    n_valid = int((ids[:, 1:] != -100).sum())
    before = logits.clone()
    buf = ops.ce_grad_buffer(logits, 2) if out_of_place else logits.clone()
    src = logits if out_of_place else buf
    loss, ws = ops.cross_entropy_shifted(src, ids, write_grad=True,
                                         grad=buf if out_of_place else None)
    assert abs(loss.item() - ref_loss.item()) <= t_ce.LOSS_RTOL * abs(ref_loss.item())
    assert ops.cross_entropy_status(ws) == 0
    if dtype == torch.float16:
        # the deferred gradient at a GradScaler-sized scale (as in the module's _check)
        scale = t_ce._fp16_scale_for(n_valid)
        ops.cross_entropy_shifted_scale_grad(buf, ids, torch.full((), scale, device=gpu), workspace=ws,
                                             logits=logits if out_of_place else None)
        t_ce._fp16_grad_close(buf, ref_grad, scale, n_valid)
    else:
        t_ce._grad_close(buf, ref_grad, n_valid, dtype)
    assert torch.equal(logits, before)


@pytest.mark.parametrize("case", range(CASES // 2))
def test_adamw_random_parameter_lists(gpu, case):
    rng = _rng("adamw", case)
    count = _log_uniform(rng, 1, 400)
    sizes = [_log_uniform(rng, 1, 300_000) for _ in range(count)]
    clip = bool(rng.integers(2))
    hp = dict(lr=float(rng.uniform(1e-4, 1e-2)), betas=(0.9, float(rng.uniform(0.9, 0.999))),
              eps=1e-8, weight_decay=float(rng.uniform(0.0, 0.2)))
    print(f"adamw case {case}: {count} tensors, {sum(sizes)} elements, clip {clip}, {hp}", flush=True)
    seed = 7000 + 1000 * case
    fused = [torch.nn.Parameter(randn((n,), torch.float32, gpu, seed + i, 0.02)) for i, n in enumerate(sizes)]
    ref = [torch.nn.Parameter(p.detach().clone()) for p in fused]
    initial = [float(p.detach().abs().max()) for p in fused]
    opt_f = torch.optim.AdamW(fused, **hp)
    opt_r = torch.optim.AdamW(ref, foreach=False, **hp)
    for step in range(2):
        for i, (a, r) in enumerate(zip(fused, ref)):
            grad = randn(a.shape, torch.float32, gpu, seed + 500 + 7 * i + step, 1e-3)
            a.grad, r.grad = grad, grad.clone()
        if clip:
            total = triton_clip_grad_norm_and_step(opt_f, 0.05)
            close_fp32(total.reshape(()), torch.nn.utils.clip_grad_norm_(ref, 0.05).reshape(()))
        else:
            triton_adamw_step(opt_f)
        opt_r.step()
    # A parameter is its initial value minus two updates of about lr each, and exp_avg a sum
    # of (1 - beta1) * g terms (g ~ 1e-3): either can nearly cancel in a small tensor, so their
    # absolute floor scales with those summands (the clip coefficient, from a differently
    # ordered fp32 norm, moves every update in its last bits).  exp_avg_sq sums squares.
    for a, r, p0 in zip(fused, ref, initial):
        close_fp32(a.detach(), r.detach(), scale=max(p0, 2 * hp["lr"], float(r.detach().abs().max())))
        m = opt_r.state[r]["exp_avg"]
        close_fp32(opt_f.state[a]["exp_avg"], m, scale=max(1e-4, float(m.abs().max())))
        close_fp32(opt_f.state[a]["exp_avg_sq"], opt_r.state[r]["exp_avg_sq"])
