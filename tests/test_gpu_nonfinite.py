"""Non-finite inputs -- an fp16 overflow upstream, a NaN -- reach the outputs and gradients
where the reference's PyTorch paths put them, so that a GradScaler sees the overflow and a
row that holds none is untouched: for each op, the finite / non-finite pattern of every
output and gradient matches the reference fallback's (oracle/*.fallback_forward_backward,
the reference code as it runs), and the finite values match to the dtype's tolerance."""

from __future__ import annotations

import pytest
import torch

from gpu_util import randn
from oracle import rmsnorm as o_rms
from oracle import rope as o_rope
from oracle import swiglu as o_swiglu
from picotron_amd import ops

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.bfloat16: dict(rtol=1.6e-2, atol=2e-2),
       torch.float16: dict(rtol=2e-3, atol=2e-3)}
BAD = [float("inf"), float("-inf"), float("nan")]


def _same(got, want, dtype, name):
    g, w = got.float(), want.float().to(got.device)
    fin = torch.isfinite(w)
    assert torch.equal(torch.isfinite(g), fin), (
        f"{name}: non-finite at {torch.nonzero(~torch.isfinite(g))[:8].tolist()}, "
        f"reference at {torch.nonzero(~fin)[:8].tolist()}")
    torch.testing.assert_close(g[fin], w[fin], **TOL[dtype], msg=name)


@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, 4096), (torch.float32, 1024), (torch.float16, 2000)])
@pytest.mark.parametrize("bad", BAD)
@pytest.mark.parametrize("where", ["x", "dy"])
def test_rmsnorm(gpu, dtype, cols, bad, where):
    x = randn((6, cols), dtype, gpu, 1, 1.0)
    w = randn((cols,), torch.float32, gpu, 2, 0.1, 1.0)
    dy = randn((6, cols), dtype, gpu, 3, 1.0)
    (x if where == "x" else dy)[1, 7] = bad
    y, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    dx, dw = ops.rmsnorm_bwd(dy, x, w, rstd)
    y_r, rstd_r, dx_r, dw_r = o_rms.fallback_forward_backward(x, w, 1e-5, dy)
    _same(y, y_r, dtype, "y")
    _same(rstd, rstd_r, torch.float32, "rstd")
    _same(dx, dx_r, dtype, "dx")
    # every row but the bad one is untouched by it
    assert bool(torch.isfinite(dx[[0, 2, 3, 4, 5]]).all())
    # the weight gradient sums over rows in another order: fp32 accumulation tolerance
    fin = torch.isfinite(dw_r)
    assert torch.equal(torch.isfinite(dw), fin)
    torch.testing.assert_close(dw[fin], dw_r[fin], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bad", BAD)
@pytest.mark.parametrize("where", ["x", "residual", "dy", "dh_in"])
def test_residual_rmsnorm(gpu, dtype, bad, where):
    """The residual add fused into the norm: h = x + residual carries a bad value into the
    norm, dh_in adds after it; the reference is the add, then the norm's PyTorch path, with
    dh_in added to its input gradient."""

    cols = 4096
    x = randn((6, cols), dtype, gpu, 11, 1.0)
    res = randn((6, cols), dtype, gpu, 12, 1.0)
    w = randn((cols,), torch.float32, gpu, 13, 0.1, 1.0)
    dy = randn((6, cols), dtype, gpu, 14, 1.0)
    dh_in = randn((6, cols), dtype, gpu, 15, 1.0)
    {"x": x, "residual": res, "dy": dy, "dh_in": dh_in}[where][1, 7] = bad
    h, y, rstd = ops.residual_rmsnorm_fwd(x, res, w, 1e-5)
    dh, dw = ops.residual_rmsnorm_bwd(dy, dh_in, h, w, rstd)
    h_r = (x.float() + res.float()).to(dtype)
    y_r, rstd_r, dx_r, dw_r = o_rms.fallback_forward_backward(h_r, w, 1e-5, dy)
    dh_r = (dx_r.float() + dh_in.float()).to(dtype)
    _same(h, h_r, dtype, "h")
    _same(y, y_r, dtype, "y")
    _same(rstd, rstd_r, torch.float32, "rstd")
    # the kernel adds dh_in before its single rounding; the reference rounds twice
    fin = torch.isfinite(dh_r.float())
    assert torch.equal(torch.isfinite(dh.float()), fin)
    torch.testing.assert_close(dh.float()[fin], dh_r.float()[fin], rtol=2 * TOL[dtype]["rtol"],
                               atol=2 * TOL[dtype]["atol"])
    assert bool(torch.isfinite(dh[[0, 2, 3, 4, 5]].float()).all())
    fin = torch.isfinite(dw_r)
    assert torch.equal(torch.isfinite(dw), fin)
    torch.testing.assert_close(dw[fin], dw_r[fin], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("bad", BAD)
@pytest.mark.parametrize("where", ["gate", "up", "dy"])
def test_swiglu(gpu, dtype, bad, where):
    n = 4099
    g = randn((n,), dtype, gpu, 4, 2.0)
    u = randn((n,), dtype, gpu, 5, 1.0)
    dy = randn((n,), dtype, gpu, 6, 1.0)
    {"gate": g, "up": u, "dy": dy}[where][[0, 1000, 4098]] = bad
    y = ops.swiglu_fwd(g, u)
    dg, du = ops.swiglu_bwd(dy, g, u)
    # the reference's path in fp32 (its ops in bf16 / fp16 round every step), then the
    # storage type
    y_r, dg_r, du_r = o_swiglu.fallback_forward_backward(g.float(), u.float(), dy.float())
    _same(y, y_r.to(dtype), dtype, "y")
    _same(dg, dg_r.to(dtype), dtype, "dgate")
    _same(du, du_r.to(dtype), dtype, "dup")


@pytest.mark.parametrize("layout", ["interleaved", "rotate_half"])
@pytest.mark.parametrize("bad", BAD)
def test_rope(gpu, layout, bad):
    b, h, s, d = 2, 3, 17, 64
    x = randn((b, h, s, d), torch.bfloat16, gpu, 7, 1.0)
    x[0, 1, 0, 5] = bad   # position 0: sin = 0, cos = 1
    x[1, 2, 9, 40] = bad
    cos, sin = o_rope.tables(s, d, 10_000.0, device=gpu)
    y, _ = ops.rope(x, cos, sin, layout=layout)
    back, _ = ops.rope(y, cos, sin, layout=layout, inverse=True)
    want = o_rope.rotate(x, cos, sin, layout, compute=torch.float32)
    _same(y, want.to(torch.bfloat16), torch.bfloat16, "y")
    want_back = o_rope.rotate(y, cos, sin, layout, inverse=True, compute=torch.float32)
    _same(back, want_back.to(torch.bfloat16), torch.bfloat16, "inverse")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bad", BAD)
def test_cross_entropy(gpu, dtype, bad):
    """A +inf or NaN logit makes its row's loss and gradient non-finite, as torch's, and so
    the mean loss; a -inf logit is a masked class (finite loss, zero gradient there).
    Every other row's gradient is untouched either way."""

    logits = randn((5, 1003), dtype, gpu, 8, 2.0)
    logits[2, 17] = bad
    targets = torch.tensor([0, 5, 9, 1002, 400], device=gpu)
    ref = logits.float().detach().requires_grad_(True)
    loss_r = torch.nn.functional.cross_entropy(ref, targets)
    loss_r.backward()
    buf = logits.clone()
    loss, ws = ops.cross_entropy(buf, targets, write_grad=True)
    assert torch.isfinite(loss).item() == torch.isfinite(loss_r).item() == (bad == float("-inf"))
    if bad == float("-inf"):
        assert abs(loss.item() - loss_r.item()) <= 1e-4 * abs(loss_r.item())
        assert float(buf[2, 17]) == 0.0
    assert torch.equal(torch.isfinite(buf.float()), torch.isfinite(ref.grad))
    assert bool(torch.isfinite(buf[[0, 1, 3, 4]].float()).all())
