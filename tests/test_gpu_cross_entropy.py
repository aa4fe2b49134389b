"""Fused cross-entropy parity of the HIP kernels (through the C ABI) with the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import GOLDEN
from gpu_util import from_npz, randn
from oracle import cross_entropy as o_ce
from picotron_amd import ops

pytestmark = pytest.mark.gpu

LOSS_RTOL = 1e-4  # fp32-accumulated loss vs the fp64 oracle

# fp32 target entries softmax_t - 1 (the negative entries of the gradient): for a dominant
# target the difference cancels, and its error is that of softmax_t rounded near 1, a few
# units of 2^-24, not relative to the small difference (torch's fp32 exp(log_softmax_t) - 1
# cancels the same way).  Observed up to 8.4e-8 over 2200 random shapes (vocab 2 rows, where
# targets often dominate); the bound is 8 units.
TARGET_ATOL_FP32 = 2.0**-21


def _grad_close(grad, ref, n_valid, dtype):
    # d loss/d logits = (softmax - onehot) / n_valid: compare (softmax - onehot) so the
    # relative tolerance of the storage type applies to O(1/V)..O(1) values.  fp16 gradients
    # exist only at a loss scale and are checked there (_fp16_grad_close).
    assert dtype in (torch.float32, torch.bfloat16), "fp16 gradients: use _fp16_grad_close"
    rtol = {torch.float32: 1e-5, torch.bfloat16: 1.6e-2}[dtype]
    atol = {torch.float32: 1e-9, torch.bfloat16: 1e-7}[dtype]
    a, e = grad.double() * n_valid, ref.double() * n_valid
    if dtype == torch.float32 and e.numel() > 0:
        tol = rtol * e.abs() + torch.where(e < 0, TARGET_ATOL_FP32, atol)
        excess = (a - e).abs() - tol
        worst = int(excess.argmax())
        assert float(excess.flatten()[worst]) <= 0, (
            f"fp32 gradient entry {worst}: {float(a.flatten()[worst])} against "
            f"{float(e.flatten()[worst])} (tolerance {float(tol.flatten()[worst])})")
    else:
        torch.testing.assert_close(a, e, rtol=rtol, atol=atol)


def _fp16_scale_for(n_valid: int) -> float:
    """A GradScaler-sized loss gradient: the initial 2^16, halved for a single valid row,
    whose target entry (softmax_t - 1) * g would otherwise round past fp16's largest finite
    value (in torch's path as well: GradScaler would then back off)."""

    return 65536.0 if n_valid > 1 else 32768.0


def _fp16_grad_close(grad, ref_grad, scale, n_valid):
    # fp16 gradient written at a loss scale: relative bound 2e-3 with a floor of one fp16
    # subnormal step (2^-24), independent of the row count.  A target entry is computed in
    # fp32 as softmax_t - 1 before it is scaled and rounded, so it carries the same absolute
    # cancellation error as the fp32 gradient's target entries (TARGET_ATOL_FP32), times
    # scale / n_valid: seen at a dominant target of a vocabulary-2 row (1.9e-5 past the
    # relative bound, within this term's 5e-5).
    ref = ref_grad.to(grad.device).double() * scale
    target = torch.where(ref < 0, TARGET_ATOL_FP32 * scale / n_valid, 0.0)
    excess = (grad.double() - ref).abs() - (2e-3 * ref.abs() + 2.0 ** -24 + target)
    assert float(excess.max()) <= 0, f"fp16 gradient: max excess {float(excess.max())}"


def _loss_only_streams(logits, dtype) -> bool:
    """Whether the loss-only forward takes the read-only streaming kernel, while a forward
    that writes the gradient takes another one: rows (aligned or not) below 2 GB."""

    return logits.size(-1) * logits.element_size() + 256 * 8 * 16 < 2**31


def _check(logits, targets, dtype):
    ref_loss, ref_grad = o_ce.forward_backward(logits, targets)
    n_valid = int((targets != -100).sum())
    loss, ws = ops.cross_entropy(logits, targets)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    buf = logits.clone()
    loss2, ws = ops.cross_entropy(buf, targets, write_grad=True)
    # the kernels split rows at 128-byte lines, so a copy at another phase of a line sums
    # in another order
    same_split = (buf.data_ptr() - logits.data_ptr()) % 128 == 0
    if (dtype == torch.float16 or not _loss_only_streams(logits, dtype)) and same_split:
        # the same kernel with and without the gradient (fp16 defers it to the backward)
        assert loss2.item() == loss.item()
    else:
        # fp32 / bf16: the kernel that writes the gradient in place against the read-only
        # streaming pass of the loss alone: the same sum in another order
        assert abs(loss2.item() - loss.item()) <= 1e-6 * abs(loss.item())
    assert ops.cross_entropy_status(ws) == 0
    if dtype == torch.float16:
        # the fp16 forward leaves the logits alone; the backward writes the gradient.  A
        # GradScaler-sized loss gradient keeps it representable (at a grad_output of 1,
        # softmax / n_valid is mostly below fp16's subnormals in the reference as well):
        # relative bound with a floor of one fp16 subnormal step, independent of n_valid
        assert torch.equal(buf, logits)
        g = _fp16_scale_for(n_valid)
        ops.cross_entropy_scale_grad(buf, targets, torch.full((), g, device=logits.device), workspace=ws)
        _fp16_grad_close(buf, ref_grad, g, n_valid)
    else:
        # the backward for a grad_output of 1 leaves fp32 / bf16 rows as the forward wrote them
        ops.cross_entropy_scale_grad(buf, targets, torch.ones((), device=logits.device), workspace=ws)
        _grad_close(buf, ref_grad, n_valid, dtype)
    return buf


def test_reference_known_answer(gpu):
    f = np.load(GOLDEN / "cross_entropy_reference_kat.npz")
    logits = from_npz(f["logits"], gpu)
    targets = from_npz(f["targets"], gpu)
    loss, _ = ops.cross_entropy(logits, targets)
    assert abs(loss.item() - 1.2887259920) < 1e-6
    buf = logits.clone()
    ops.cross_entropy(buf, targets, write_grad=True)
    torch.testing.assert_close(buf, from_npz(f["grad"], gpu), rtol=1e-5, atol=1e-7)


def test_golden_fixture(gpu):
    f = np.load(GOLDEN / "cross_entropy_small.npz")
    logits = from_npz(f["logits"], gpu)
    targets = from_npz(f["targets"], gpu)
    loss, _ = ops.cross_entropy(logits, targets)
    assert abs(loss.item() - float(f["loss"])) <= 1e-5 * abs(float(f["loss"]))
    buf = logits.clone()
    ops.cross_entropy(buf, targets, write_grad=True)
    _grad_close(buf, from_npz(f["grad"], gpu), 13, torch.float32)


def test_full_config_bf16(gpu):
    # logits [8192, 128256] bf16 ~ N(0, 2^2); targets uniform, exactly 410 (5%) ignored
    rows, vocab = 8192, 128256
    logits = randn((rows, vocab), torch.bfloat16, gpu, 51, 2.0)
    g = torch.Generator(device=gpu).manual_seed(52)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    targets[torch.randperm(rows, generator=g, device=gpu)[:410]] = -100
    ref_loss, ref_grad = o_ce.forward_backward(logits, targets)
    loss, ws = ops.cross_entropy(logits, targets, write_grad=True)  # in place
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    assert ops.cross_entropy_status(ws) == 0
    _grad_close(logits, ref_grad, rows - 410, torch.bfloat16)
    # size-independent: every kept row of (softmax - onehot) sums to 0, ignored rows are 0
    row_sums = logits.double().sum(-1) * (rows - 410)
    assert float(row_sums.abs().max()) < 5e-3
    assert bool((logits[targets == -100] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "rows,vocab",
    [(1, 1), (5, 3), (7, 1000), (33, 8192), (4, 50257), (3, 131072), (3, 151936), (2, 248320), (2, 262144)],
)
def test_shapes(gpu, dtype, rows, vocab):
    logits = randn((rows, vocab), dtype, gpu, rows * 3 + vocab, 2.0)
    g = torch.Generator(device=gpu).manual_seed(vocab)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    if rows > 2:
        targets[1] = -100
    _check(logits, targets, dtype)


@pytest.mark.parametrize(
    "dtype,vocab",
    [(torch.bfloat16, 24), (torch.bfloat16, 50264), (torch.float16, 50264), (torch.bfloat16, 128256),
     (torch.float16, 128256), (torch.float32, 65528), (torch.float32, 12), (torch.bfloat16, 151936),
     (torch.float16, 151936), (torch.bfloat16, 262144), (torch.float32, 65540)],
)
def test_targets_at_the_ends_of_ragged_register_rows(gpu, dtype, vocab):
    # 16-byte aligned rows (held in registers, or streamed in batches when longer) whose last
    # chunk of vectors is only partly inside the row: targets at the first and last logit,
    # at the first element of the last chunk and of the vector before it, and an ignored row.
    v = 16 // torch.tensor([], dtype=dtype).element_size()
    per_thread = -(-vocab // (1024 * v))  # chunks of 1024 vectors that hold logits
    last_chunk = (per_thread - 1) * 1024 * v  # first logit of the chunk holding the last one
    picks = [0, vocab - 1, last_chunk, max(last_chunk - v, 0), -100, vocab // 2]
    # every target is a valid index (the oracle's gather on the GPU does not check bounds)
    assert all(p == -100 or 0 <= p < vocab for p in picks)
    logits = randn((len(picks), vocab), dtype, gpu, vocab + 11, 2.0)
    targets = torch.tensor(picks, device=gpu)
    _check(logits, targets, dtype)


def _line_split_targets(logits, rows, vocab, es):
    """Per row, a target on one side of the row's splits: its head (the elements before its
    first 128-byte line), its body of 16-byte vectors from that line and its tail."""

    v = 16 // es
    picks = []
    for r in range(rows):
        addr = logits.data_ptr() + r * logits.stride(0) * es
        head = min(((128 - addr % 128) % 128) // es, vocab)
        tail_start = head + (vocab - head) // v * v
        candidates = [c for c in (head - 1, head, tail_start - 1, tail_start, 0, vocab - 1) if 0 <= c < vocab]
        picks.append(candidates[r % len(candidates)])
    return picks


@pytest.mark.parametrize(
    "dtype,vocab",
    [(torch.bfloat16, 50257), (torch.float16, 50257), (torch.float32, 1001), (torch.bfloat16, 151939),
     (torch.float16, 200003), (torch.bfloat16, 50256), (torch.float32, 32008), (torch.bfloat16, 128264)],
)
def test_targets_at_the_splits_of_unaligned_rows(gpu, dtype, vocab):
    # Rows whose byte stride is not a multiple of 128 start at varying places in a cache
    # line; each is split into a head before its first 128-byte line, a body of 16-byte
    # vectors and a tail.  Targets sit on both sides of each split and at the ends of the row.
    es = torch.tensor([], dtype=dtype).element_size()
    rows = 16
    logits = randn((rows, vocab), dtype, gpu, vocab + 13, 2.0)
    picks = _line_split_targets(logits, rows, vocab, es)
    picks[5] = -100
    assert all(p == -100 or 0 <= p < vocab for p in picks)
    _check(logits, torch.tensor(picks, device=gpu), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("vocab", [1, 7, 63, 65, 129, 1031, 9001])
@pytest.mark.parametrize("offset", [0, 1, 3, 8, 17, 31, 32, 47, 63, 64, 71])
def test_row_starts_in_every_line_phase(gpu, dtype, vocab, offset):
    """Rows cut from one flat buffer at an element offset: with an odd vocabulary the rows
    start at every phase of a 128-byte line, so heads run from none to a whole line (63
    16-bit or 31 fp32 elements) and, for short rows, past the row's end; targets sit on
    both sides of each split."""

    es = torch.tensor([], dtype=dtype).element_size()
    rows = 9
    flat = randn((offset + rows * vocab,), dtype, gpu, 1000 * vocab + offset, 2.0)
    logits = flat[offset:].view(rows, vocab)
    picks = _line_split_targets(logits, rows, vocab, es)
    picks[rows // 2] = -100
    _check(logits, torch.tensor(picks, device=gpu), dtype)


@pytest.mark.parametrize(
    "dtype,vocab",
    [(torch.bfloat16, 4096), (torch.bfloat16, 262144), (torch.float32, 1001), (torch.float16, 50257)],
)
def test_masked_logits(gpu, dtype, vocab):
    # -inf logits (masked vocabulary padding) contribute 0 to the softmax and get a zero
    # gradient; the masked tail covers whole per-thread chunks of every kernel variant.
    rows = 6
    logits = randn((rows, vocab), dtype, gpu, vocab + 7, 2.0)
    keep = vocab * 3 // 5
    logits[:, keep:] = float("-inf")
    logits[:, 1::7] = float("-inf")
    g = torch.Generator(device=gpu).manual_seed(vocab + 8)
    targets = torch.randint(0, keep, (rows,), generator=g, device=gpu)
    targets = torch.where(targets % 7 == 1, targets - 1, targets)  # never a masked target
    buf = _check(logits, targets, dtype)
    assert bool((buf[:, keep:] == 0).all())
    assert bool(torch.isfinite(buf).all())


def test_train_loop_view(gpu):
    # loss(logits[:, :-1, :].transpose(1, 2), input_ids[:, 1:]) on (B, S, V) bf16 logits
    b, s, v = 2, 65, 3000
    full = randn((b, s, v), torch.bfloat16, gpu, 61, 2.0)
    g = torch.Generator(device=gpu).manual_seed(62)
    ids = torch.randint(0, v, (b, s), generator=g, device=gpu)
    view = full[:, :-1, :].transpose(1, 2)
    targets = ids[:, 1:]
    ref_loss, ref_grad = o_ce.forward_backward(view, targets)
    last = full[:, -1, :].clone()
    loss, _ = ops.cross_entropy(view, targets, write_grad=True)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    _grad_close(view, ref_grad, b * (s - 1), torch.bfloat16)
    assert torch.equal(full[:, -1, :], last)  # the unused last position is untouched


# Two and more rows per CU (256 CUs here) of 9 to 16 vectors per thread on 128-byte lines
# (vocabularies below: multiples of 64 bf16 or 32 fp32 logits): the register rows of one
# workgroup per CU, several after one another on each CU
MANY_ROWS = 2 * 256 + 9


@pytest.mark.parametrize(
    "dtype,vocab",
    [(torch.bfloat16, 73_024), (torch.bfloat16, 90_112), (torch.bfloat16, 110_592), (torch.bfloat16, 128_256),
     (torch.bfloat16, 131_072), (torch.float32, 40_000), (torch.float32, 51_200), (torch.float32, 65_536)],
)
def test_many_long_rows(gpu, dtype, vocab):
    """Every row against the oracle, with ignored rows (zeros stored) in runs and alone, the
    last rows of the grid, and targets at the first and last logit and at the ends of the
    last chunk."""

    v = 16 // torch.tensor([], dtype=dtype).element_size()
    per_thread = -(-vocab // (1024 * v))
    last_chunk = (per_thread - 1) * 1024 * v
    logits = randn((MANY_ROWS, vocab), dtype, gpu, vocab + 31, 2.0)
    g = torch.Generator(device=gpu).manual_seed(vocab)
    targets = torch.randint(0, vocab, (MANY_ROWS,), generator=g, device=gpu)
    picks = [0, vocab - 1, last_chunk, max(last_chunk - v, 0), min(last_chunk + v - 1, vocab - 1)]
    for i, p in enumerate(picks):
        targets[i * 97 % MANY_ROWS] = p
    targets[3] = targets[255] = targets[256] = targets[257] = -100  # one row of each CU's second turn
    targets[-1] = targets[-2] = -100
    _check(logits, targets, dtype)


def test_many_long_rows_flag_a_bad_target(gpu):
    logits = randn((MANY_ROWS, 128_256), torch.bfloat16, gpu, 77, 2.0)
    targets = torch.zeros(MANY_ROWS, dtype=torch.int64, device=gpu)
    targets[300] = 128_256
    buf = logits.clone()
    loss, ws = ops.cross_entropy(buf, targets, write_grad=True)
    assert math.isnan(loss.item()) and ops.cross_entropy_status(ws) & 1


def test_ignored_rows_and_bad_targets(gpu):
    logits = randn((6, 100), torch.float32, gpu, 71)
    targets = torch.full((6,), -100, device=gpu)
    buf = logits.clone()
    loss, _ = ops.cross_entropy(buf, targets, write_grad=True)
    assert math.isnan(loss.item())  # 0 / 0, as F.cross_entropy
    assert bool((buf == 0).all())
    bad = torch.tensor([1, 100, 3, -5, 2, 0], device=gpu)
    loss, ws = ops.cross_entropy(logits, bad)
    assert math.isnan(loss.item()) and ops.cross_entropy_status(ws) & 1


def test_autograd_surface_and_grad_scaling(gpu):
    import warnings

    from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback, triton_cross_entropy

    full = randn((2, 33, 500), torch.bfloat16, gpu, 81, 2.0)
    g = torch.Generator(device=gpu).manual_seed(82)
    ids = torch.randint(0, 500, (2, 33), generator=g, device=gpu)
    ids[0, 5] = -100
    ref_loss, ref_grad = o_ce.forward_backward(full[:, :-1, :].transpose(1, 2), ids[:, 1:])
    leaf = full.clone().requires_grad_(True)
    logits = leaf * 1  # non-leaf, as a projection output
    ce = CrossEntropyWithFallback(use_triton=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        loss = ce(logits[:, :-1, :].transpose(1, 2), ids[:, 1:])
    assert not ce._fallback_warned
    assert loss.dtype == torch.float32
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    (3.0 * loss).backward()  # grad_output != 1 takes the on-device scaling path
    n_valid = int((ids[:, 1:] != -100).sum())
    expected = torch.zeros_like(full, dtype=torch.float64)
    expected[:, :-1, :] = 3.0 * ref_grad.transpose(1, 2)
    _grad_close(leaf.grad, expected, n_valid, torch.bfloat16)
    # inplace=False keeps the logits intact
    x = full.clone().requires_grad_(True)
    y = x * 1
    loss2 = triton_cross_entropy(y[:, :-1, :].transpose(1, 2), ids[:, 1:], inplace=False)
    assert torch.equal(y.detach(), full)
    loss2.backward()
    _grad_close(x.grad, expected / 3.0, n_valid, torch.bfloat16)


def _shifted_case(gpu, b, s, v, dtype, seed):
    logits = randn((b, s, v), dtype, gpu, seed, 2.0)
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    ids = torch.randint(0, v, (b, s), generator=g, device=gpu)
    if s > 3:
        ids[0, 2] = -100
        ids[-1, -1] = -100
    return logits, ids


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,s,v", [(2, 65, 3000), (3, 17, 50257), (1, 9, 1001), (2, 2, 128), (2, 33, 32001)])
def test_shifted_matches_the_train_loop_expression(gpu, dtype, b, s, v):
    logits, ids = _shifted_case(gpu, b, s, v, dtype, 7 * s + v)
    ref_loss, ref_grad = o_ce.shifted_forward_backward(logits, ids)
    n_valid = int((ids[:, 1:] != -100).sum())
    loss, ws = ops.cross_entropy_shifted(logits, ids)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    view_loss, _ = ops.cross_entropy(logits[:, :-1, :].transpose(1, 2), ids[:, 1:])
    assert abs(loss.item() - view_loss.item()) <= 1e-6 * abs(view_loss.item())
    buf = logits.clone()
    loss2, ws = ops.cross_entropy_shifted(buf, ids, write_grad=True)
    if dtype == torch.float16 and (buf.data_ptr() - logits.data_ptr()) % 128 == 0:
        assert loss2.item() == loss.item()  # one read-only kernel (the gradient is deferred)
    else:
        # the kernel that writes the gradient against the read-only pass: another sum order
        assert abs(loss2.item() - loss.item()) <= 1e-6 * abs(loss.item())
    assert ops.cross_entropy_status(ws) == 0
    if dtype == torch.float16:
        # the deferred gradient, written by the backward at a GradScaler-sized scale (odd
        # vocabularies: the unaligned rows' head / body / tail split)
        assert torch.equal(buf, logits)
        scale = _fp16_scale_for(n_valid)
        ops.cross_entropy_shifted_scale_grad(buf, ids, torch.full((), scale, device=gpu), workspace=ws)
        _fp16_grad_close(buf, ref_grad, scale, n_valid)
    else:
        _grad_close(buf, ref_grad, n_valid, dtype)
    assert bool((buf[:, -1, :] == 0).all())  # the last position has no target


def test_shifted_full_config_bf16(gpu):
    # (B, S, V) = (4, 2049, 128256) bf16: 8196 predicted positions, about the cfg5 row count
    b, s, v = 4, 2049, 128256
    logits, ids = _shifted_case(gpu, b, s, v, torch.bfloat16, 91)
    ids[1, 100:300] = -100
    n_valid = int((ids[:, 1:] != -100).sum())
    ref_loss, ref_grad = o_ce.shifted_forward_backward(logits, ids)
    loss, ws = ops.cross_entropy_shifted(logits, ids, write_grad=True)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    assert ops.cross_entropy_status(ws) == 0
    _grad_close(logits, ref_grad, n_valid, torch.bfloat16)
    del ref_grad
    row_sums = logits.double().sum(-1) * n_valid  # kept rows of softmax - onehot sum to 0
    assert float(row_sums.abs().max()) < 5e-3
    assert bool((logits[:, -1, :] == 0).all())
    assert bool((logits[1, 99:299, :] == 0).all())  # positions whose next id is ignored


def test_shifted_single_position_has_no_targets(gpu):
    logits = randn((3, 1, 64), torch.float32, gpu, 5)
    ids = torch.randint(0, 64, (3, 1), device=gpu)
    buf = logits.clone()
    loss, _ = ops.cross_entropy_shifted(buf, ids, write_grad=True)
    assert math.isnan(loss.item())  # mean over no targets, as F.cross_entropy
    assert bool((buf == 0).all())


def test_shifted_autograd_surface(gpu):
    from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback, triton_cross_entropy

    full, ids = _shifted_case(gpu, 2, 33, 500, torch.bfloat16, 83)
    ref_loss, ref_grad = o_ce.shifted_forward_backward(full, ids)
    n_valid = int((ids[:, 1:] != -100).sum())
    leaf = full.clone().requires_grad_(True)
    ce = CrossEntropyWithFallback(use_triton=True)
    loss = ce(leaf * 1, ids, shift=True)
    assert not ce._fallback_warned
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    (2.5 * loss).backward()  # grad_output != 1: on-device scaling, last position stays 0
    _grad_close(leaf.grad, 2.5 * ref_grad, n_valid, torch.bfloat16)
    assert bool((leaf.grad[:, -1, :] == 0).all())
    x = full.clone().requires_grad_(True)
    y = x * 1
    loss2 = triton_cross_entropy(y, ids, shift=True, inplace=False)
    assert torch.equal(y.detach(), full)
    loss2.backward()
    _grad_close(x.grad, ref_grad, n_valid, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("vocab", [3, 7, 8, 9, 1001, 50257])
@pytest.mark.parametrize("offset", [0, 1])
def test_scale_grad_is_the_elementwise_product(gpu, dtype, vocab, offset):
    # rows split into head / 16-byte body / tail at every alignment (row starts shifted by a
    # one-element view offset): each kept element becomes (x * scale) rounded once, bit for
    # bit; ignored rows are left alone
    rows = 11
    base = randn((rows, vocab + offset), dtype, gpu, vocab + offset)
    buf = base[:, offset:]
    targets = torch.randint(0, vocab, (rows,), device=gpu)
    targets[[2, 7]] = -100
    before = buf.clone()
    outside = base[:, :offset].clone()
    ops.cross_entropy_scale_grad(buf, targets, torch.tensor(0.37, device=gpu))
    kept = (targets != -100).unsqueeze(1)
    want = torch.where(kept, (before.float() * 0.37).to(dtype), before)
    assert torch.equal(buf, want)
    assert torch.equal(base[:, :offset], outside)  # nothing outside the view is written


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("vocab", [512, 1001, 131072])
def test_scale_grad(gpu, dtype, vocab):
    # the backward's on-device scaling, for aligned (16-byte vector) and element-wise rows;
    # ignored rows stay exactly 0 whatever the scale (NaN included)
    rows = 9
    logits = randn((rows, vocab), dtype, gpu, vocab + 3, 2.0)
    targets = torch.randint(0, vocab, (rows,), device=gpu)
    targets[4] = -100
    _, ref_grad = o_ce.forward_backward(logits, targets)
    buf = logits.clone()
    _, ws = ops.cross_entropy(buf, targets, write_grad=True)
    ops.cross_entropy_scale_grad(buf, targets, torch.tensor(0.37, device=gpu), workspace=ws)
    _grad_close(buf, 0.37 * ref_grad, rows - 1, dtype)
    ops.cross_entropy_scale_grad(buf, targets, torch.tensor(float("nan"), device=gpu), workspace=ws)
    assert bool((buf[4] == 0).all())
    assert bool(torch.isnan(buf[targets != -100]).all())


@pytest.mark.parametrize("shift", [False, True])
def test_fp16_gradients_at_training_scale(gpu, shift):
    """fp16 logits at the training shape with a GradScaler-sized loss gradient (65536).

    softmax / n_valid (about 1e-10 here) lies far below fp16's smallest subnormal, so a
    gradient stored before the scale is known would be all zeros: at least 99% of the entries
    of the rows that have a target must be nonzero.  Bounds are relative, with an absolute
    floor of fp16 subnormal steps (independent of the row count), against two references:
    - F.cross_entropy on the fp32 upcast, its gradient rounded to fp16 once (within half an
      fp16 unit of the exact gradient), as the fused backward rounds once: 1e-3 relative (one
      fp16 unit at the bottom of a binade) and one subnormal step;
    - the reference's own call, F.cross_entropy under fp16 autocast: its backward deviates from
      the exact gradient by up to 0.44% on this build (measured; an fp32 computation rounded once
      deviates by 0.05%), so 6e-3 relative and two subnormal steps.
    """

    from picotron_amd.nn.triton_kernels import triton_cross_entropy

    vocab, scale = 128256, 65536.0
    shape = (2, 1025, vocab) if shift else (8192, vocab)
    print(f"fp16 ce shape {shape} shift {shift}", flush=True)
    logits = randn(shape, torch.float16, gpu, 91, 2.0)
    g = torch.Generator(device=gpu).manual_seed(92)
    if shift:
        targets = torch.randint(0, vocab, shape[:2], generator=g, device=gpu)
        targets[0, 7:300] = -100
    else:
        targets = torch.randint(0, vocab, shape[:1], generator=g, device=gpu)
        targets[torch.randperm(shape[0], generator=g, device=gpu)[:410]] = -100

    def reference(cast_fp32: bool):
        leaf = logits.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.float16, enabled=not cast_fp32):
            t = leaf.float() if cast_fp32 else leaf
            if shift:
                loss = F.cross_entropy(t[:, :-1, :].transpose(1, 2), targets[:, 1:])
            else:
                loss = F.cross_entropy(t, targets)
        (loss * scale).backward()
        return loss.detach(), leaf.grad

    x = logits.clone().requires_grad_(True)
    loss = triton_cross_entropy(x * 1, targets, shift=shift)
    (loss * scale).backward()
    got = x.grad.float()
    assert x.grad.dtype == torch.float16
    for cast_fp32, rtol, floor in ((True, 1e-3, 2.0 ** -24), (False, 6e-3, 2.0 ** -23)):
        ref_loss, ref = reference(cast_fp32)
        assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
        ref = ref.float()
        excess = (got - ref).abs() - (rtol * ref.abs() + floor)
        assert float(excess.max()) <= 0, f"fp32-upcast reference {cast_fp32}: max excess {float(excess.max())}"
        if cast_fp32:  # over the rows that have a target (ignored rows are zero)
            kept = (targets[:, 1:] if shift else targets) != -100
            rows_got = (got[:, :-1] if shift else got)[kept]
            rows_ref = (ref[:, :-1] if shift else ref)[kept]
            nonzero = float((rows_got != 0).float().mean())
            assert nonzero > 0.99, nonzero
            assert abs(nonzero - float((rows_ref != 0).float().mean())) < 1e-3
            del rows_got, rows_ref
        del ref, excess


def test_repeated_backward_raises_clearly(gpu):
    from picotron_amd.nn.triton_kernels import triton_cross_entropy

    logits = randn((4, 300), torch.bfloat16, gpu, 93, 2.0)
    targets = torch.tensor([1, 2, -100, 299], device=gpu)
    x = logits.clone().requires_grad_(True)
    loss = triton_cross_entropy(x * 1, targets)
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="consumed by an earlier backward"):
        loss.backward()


def test_overlapping_rows_are_never_written_in_place(gpu):
    from picotron_amd.nn.triton_kernels import (
        CrossEntropyWithFallback,
        TritonCrossEntropyUnavailable,
        triton_cross_entropy,
    )

    row = randn((1, 500), torch.bfloat16, gpu, 94, 2.0).requires_grad_(True)
    expanded = row.expand(6, 500)  # six rows on one row of memory
    targets = torch.tensor([0, 1, 2, 3, -100, 499], device=gpu)
    with pytest.raises(TritonCrossEntropyUnavailable, match="overlap"):
        triton_cross_entropy(expanded, targets)
    # out of place it runs, and matches the oracle on the materialised rows
    ref_loss, ref_grad = o_ce.forward_backward(expanded.detach().contiguous(), targets)
    loss = triton_cross_entropy(expanded, targets, inplace=False)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    loss.backward()
    _grad_close(row.grad, ref_grad.sum(0, keepdim=True), 5, torch.bfloat16)
    # the drop-in keeps its input by default, like F.cross_entropy
    logits = randn((5, 700), torch.bfloat16, gpu, 95, 2.0)
    y = logits.clone().requires_grad_(True) * 1
    before = y.detach().clone()
    CrossEntropyWithFallback(use_triton=True)(y, torch.tensor([0, 5, 9, -100, 699], device=gpu)).backward()
    assert torch.equal(y.detach(), before)


@pytest.mark.parametrize("grad_output", [65536.0, 3.0])
@pytest.mark.parametrize(
    "vocab,offset", [(1000, 0), (50257, 0), (50257, 1), (131072, 0), (151936, 0), (151936, 3)]
)
def test_fp16_gradient_is_written_by_the_backward(gpu, vocab, offset, grad_output):
    """fp16: the forward leaves the logits alone and keeps each row's log-sum-exp; the
    backward writes (softmax - onehot) * grad_output / n_valid rounded once, on aligned rows
    (the read-only streaming forward) and unaligned ones (row starts shifted by an element
    offset: the batched forward), short and long, with targets at
    both ends of the row and an ignored row; nothing outside the view is written."""

    rows = 12
    base = randn((rows, vocab + offset), torch.float16, gpu, vocab + 17 * offset, 2.0)
    logits = base[:, offset:]
    g = torch.Generator(device=gpu).manual_seed(vocab + offset)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    targets[3], targets[5], targets[7] = -100, vocab - 1, 0
    before = logits.clone()
    outside = base[:, :offset].clone()
    loss, ws = ops.cross_entropy(logits, targets, write_grad=True)
    ref_loss, ref_grad = o_ce.forward_backward(before, targets)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    assert torch.equal(logits, before)
    ops.cross_entropy_scale_grad(logits, targets, torch.tensor(grad_output, device=gpu), workspace=ws)
    want = ref_grad.to(gpu) * grad_output
    excess = (logits.double() - want).abs() - (1e-3 * want.abs() + 2.0 ** -24)
    assert float(excess.max()) <= 0, float(excess.max())
    assert bool((logits[3] == 0).all())
    assert torch.equal(base[:, :offset], outside)


# ------------------------------------------------------------------ gradient out of place


def _graph_names(fn, depth=6):
    names, frontier = [], [fn]
    for _ in range(depth):
        nxt = []
        for f in frontier:
            if f is None:
                continue
            names.append(type(f).__name__)
            nxt.extend(n for n, _ in f.next_functions)
        frontier = nxt
    return names


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "rows,vocab,offset",
    [(33, 8192, 0), (16, 50257, 0), (16, 50257, 1), (5, 131072, 0), (3, 151936, 0), (7, 1001, 3)],
)
def test_out_of_place_gradient_matches_in_place_bitwise(gpu, dtype, rows, vocab, offset):
    # The gradient goes to a buffer of the logits' layout (same 16-byte phase row by row) and
    # the logits are only read: the same bits as the in-place path on a copy of the logits in
    # the same layout, the logits unchanged, and the oracle's values.
    flat = randn((rows * vocab + offset,), dtype, gpu, rows + vocab + offset, 2.0)
    logits = flat[offset:].view(rows, vocab)
    g = torch.Generator(device=gpu).manual_seed(vocab + 1)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    targets[1] = -100
    before = logits.clone()
    n_valid = rows - 1
    ref_loss, ref_grad = o_ce.forward_backward(logits, targets)
    grad = ops.ce_grad_buffer(logits)
    assert (grad.data_ptr() - logits.data_ptr()) % 128 == 0 and grad.stride() == logits.stride()
    loss, ws = ops.cross_entropy(logits, targets, write_grad=True, grad=grad)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    assert ops.cross_entropy_status(ws) == 0
    same = ops.ce_grad_buffer(logits)
    same.copy_(before)
    loss_ip, ws_ip = ops.cross_entropy(same, targets, write_grad=True)
    assert loss_ip.item() == loss.item()
    scale = _fp16_scale_for(n_valid) if dtype == torch.float16 else 0.37
    go = torch.full((), scale, device=gpu)
    if dtype == torch.float16:
        assert torch.equal(logits, before)  # the forward wrote nothing
        ops.cross_entropy_scale_grad(grad, targets, go, workspace=ws, logits=logits)
        ops.cross_entropy_scale_grad(same, targets, go, workspace=ws_ip)
        _fp16_grad_close(grad, ref_grad, scale, n_valid)
    else:
        ops.cross_entropy_scale_grad(grad, targets, go, workspace=ws)
        ops.cross_entropy_scale_grad(same, targets, go, workspace=ws_ip)
        _grad_close(grad, scale * ref_grad, n_valid, dtype)
    assert torch.equal(grad, same)
    assert torch.equal(logits, before)


def test_out_of_place_full_config_bf16(gpu):
    rows, vocab = 8192, 128256
    logits = randn((rows, vocab), torch.bfloat16, gpu, 51, 2.0)
    g = torch.Generator(device=gpu).manual_seed(52)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=gpu)
    targets[torch.randperm(rows, generator=g, device=gpu)[:410]] = -100
    ref_loss, ref_grad = o_ce.forward_backward(logits, targets)
    digest_before = logits.view(torch.int16).sum(dtype=torch.int64).item()
    grad = ops.ce_grad_buffer(logits)
    loss, ws = ops.cross_entropy(logits, targets, write_grad=True, grad=grad)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    _grad_close(grad, ref_grad, rows - 410, torch.bfloat16)
    assert logits.view(torch.int16).sum(dtype=torch.int64).item() == digest_before
    del ref_grad
    ref_loss2, _ = o_ce.forward_backward(logits[:64], targets[:64])  # the logits are still the logits
    loss2, _ = ops.cross_entropy(logits[:64], targets[:64])
    assert abs(loss2.item() - ref_loss2.item()) <= LOSS_RTOL * abs(ref_loss2.item())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,s,v", [(2, 65, 3000), (3, 17, 50257), (1, 9, 1001), (2, 2, 128)])
def test_reference_call_site_unchanged(gpu, dtype, b, s, v):
    # The train loop's own call, CrossEntropyWithFallback(...)(logits[:, :-1, :].transpose(1, 2),
    # input_ids[:, 1:]) with the default inplace=False, is computed on the view's base: the
    # logits stay untouched, the graph holds no slice or transpose backward, and the base's
    # gradient (last position zero) matches the oracle.
    import warnings

    from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback

    full, ids = _shifted_case(gpu, b, s, v, dtype, 11 * s + v)
    n_valid = int((ids[:, 1:] != -100).sum())
    ref_loss, ref_grad = o_ce.shifted_forward_backward(full, ids)
    leaf = full.clone().requires_grad_(True)
    logits = leaf * 1  # non-leaf, as the language-model head's output
    before = logits.detach().clone()
    ce = CrossEntropyWithFallback(use_triton=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        loss = ce(logits[:, :-1, :].transpose(1, 2), ids[:, 1:])
    names = _graph_names(loss.grad_fn)
    assert not any("Slice" in n or "Transpose" in n for n in names), names
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    scale = _fp16_scale_for(n_valid) if dtype == torch.float16 else 2.5
    (scale * loss).backward()
    assert torch.equal(logits.detach(), before)
    if dtype == torch.float16:
        _fp16_grad_close(leaf.grad, ref_grad, scale, n_valid)
    else:
        _grad_close(leaf.grad, scale * ref_grad, n_valid, dtype)
    assert bool((leaf.grad[:, -1, :] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_other_views_take_the_generic_out_of_place_path(gpu, dtype):
    # logits[:, 1:, :].transpose(1, 2) is not the train loop's view: the loss runs on the view
    # itself, its gradient goes to a buffer of the view's layout, and autograd's slice
    # backward places it; the logits stay untouched.
    from picotron_amd.nn.triton_kernels import triton_cross_entropy

    full, ids = _shifted_case(gpu, 2, 40, 1001, dtype, 97)
    view_ref = full[:, 1:, :].transpose(1, 2)
    targets = ids[:, :-1]
    ref_loss, ref_grad = o_ce.forward_backward(view_ref, targets)
    n_valid = int((targets != -100).sum())
    leaf = full.clone().requires_grad_(True)
    logits = leaf * 1
    before = logits.detach().clone()
    loss = triton_cross_entropy(logits[:, 1:, :].transpose(1, 2), targets, inplace=False)
    assert abs(loss.item() - ref_loss.item()) <= LOSS_RTOL * abs(ref_loss.item())
    scale = _fp16_scale_for(n_valid) if dtype == torch.float16 else 1.0
    (scale * loss).backward()
    assert torch.equal(logits.detach(), before)
    expected = torch.zeros(full.shape, dtype=torch.float64, device=gpu)
    expected[:, 1:, :] = ref_grad.to(gpu).transpose(1, 2)
    if dtype == torch.float16:
        _fp16_grad_close(leaf.grad, expected, scale, n_valid)
    else:
        _grad_close(leaf.grad, expected, n_valid, dtype)
