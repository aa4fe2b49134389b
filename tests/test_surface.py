"""The reference's hot-path tests, run against this package's drop-in surface on CPU
(reference tests/test_triton_{rmsnorm_backward,swiglu_backward,rmsnorm_swiglu_rope,kernels,
ce_adamw}.py and tests/test_rope.py).  On CPU every fused path must raise its
``*Unavailable`` exception and the modules must warn once and fall back."""

from __future__ import annotations

import warnings

import pytest
import torch
from torch.nn import functional as F
from torch.optim import AdamW

from picotron_amd.config import ConfigValidationError, TritonKernelsConfig
from picotron_amd.hardware import detect_triton_support, kernel_status_rows
from picotron_amd.nn import RMSNorm, RotaryEmbedding, SwiGLU, apply_rotary_embedding, rotary_cos_sin
from picotron_amd.nn.rope import apply_rotary_embedding_rotate_half
from picotron_amd.nn.triton_kernels import (
    AdamWStepWithFallback,
    CrossEntropyWithFallback,
    TritonAdamWUnavailable,
    TritonAttentionUnavailable,
    TritonCrossEntropyUnavailable,
    TritonRMSNormUnavailable,
    TritonRoPEUnavailable,
    TritonSwiGLUUnavailable,
    rms_norm_with_pytorch_forward,
    swiglu_with_pytorch_forward,
    triton_adamw_step,
    triton_grad_scaler_step,
    triton_apply_rotary_embedding,
    triton_causal_attention,
    triton_cross_entropy,
    triton_rms_norm,
    triton_swiglu,
)


def test_public_names_match_reference_all():
    import picotron_amd.nn.triton_kernels as tk

    reference_all = {
        "AdamWStepWithFallback", "CrossEntropyWithFallback", "TritonAttentionUnavailable",
        "TritonAdamWUnavailable", "TritonCrossEntropyUnavailable", "TritonRMSNormUnavailable",
        "TritonRoPEUnavailable", "TritonSwiGLUUnavailable", "triton_causal_attention",
        "triton_apply_rotary_embedding", "triton_cross_entropy", "triton_rms_norm",
        "triton_swiglu", "swiglu_with_pytorch_forward", "rms_norm_with_pytorch_forward",
    }
    assert reference_all <= set(tk.__all__)
    for exc in (TritonAdamWUnavailable, TritonAttentionUnavailable, TritonCrossEntropyUnavailable,
                TritonRMSNormUnavailable, TritonRoPEUnavailable, TritonSwiGLUUnavailable):
        assert issubclass(exc, RuntimeError)


def test_custom_rmsnorm_backward_matches_native_rmsnorm():
    torch.manual_seed(23)
    eps = 1e-6
    upstream = torch.randn(2, 3, 8, dtype=torch.float32)
    x = torch.randn(2, 3, 8, dtype=torch.float32, requires_grad=True)
    w = torch.randn(8, dtype=torch.float32, requires_grad=True)
    out = rms_norm_with_pytorch_forward(x, w, eps)
    (out * upstream).sum().backward()
    xn = x.detach().clone().requires_grad_(True)
    wn = w.detach().clone().requires_grad_(True)
    native = xn * torch.rsqrt(xn.square().mean(dim=-1, keepdim=True) + eps) * wn
    (native * upstream).sum().backward()
    torch.testing.assert_close(out, native, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(x.grad, xn.grad, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(w.grad, wn.grad, rtol=1e-5, atol=1e-6)


def test_custom_swiglu_backward_matches_native_pytorch():
    torch.manual_seed(31)
    upstream = torch.randn(2, 3, 7, dtype=torch.float64)
    g = torch.randn(2, 3, 7, dtype=torch.float64, requires_grad=True)
    u = torch.randn(2, 3, 7, dtype=torch.float64, requires_grad=True)
    out = swiglu_with_pytorch_forward(g, u)
    (out * upstream).sum().backward()
    gn = g.detach().clone().requires_grad_(True)
    un = u.detach().clone().requires_grad_(True)
    (F.silu(gn) * un * upstream).sum().backward()
    torch.testing.assert_close(out, F.silu(gn) * un, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(g.grad, gn.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(u.grad, un.grad, rtol=1e-10, atol=1e-10)


def test_fused_entry_points_raise_unavailable_on_cpu():
    x = torch.randn(2, 3, 8)
    with pytest.raises(TritonRMSNormUnavailable):
        triton_rms_norm(x, torch.ones(8), 1e-6)
    with pytest.raises(TritonSwiGLUUnavailable):
        triton_swiglu(x, x)
    cos, sin = rotary_cos_sin(3, 8, 1e4, device=x.device, dtype=torch.float32)
    with pytest.raises(TritonRoPEUnavailable):
        triton_apply_rotary_embedding(torch.randn(2, 4, 3, 8), cos, sin)
    with pytest.raises(TritonCrossEntropyUnavailable):
        triton_cross_entropy(torch.randn(4, 5), torch.tensor([0, 1, 2, 3]))
    with pytest.raises(TritonAttentionUnavailable):
        triton_causal_attention(x, x, x)


def test_triton_enabled_cpu_fallbacks_match_native_pytorch():
    hidden = torch.randn(2, 3, 8)
    norm = RMSNorm(8, use_triton_rmsnorm=True)
    with pytest.warns(RuntimeWarning, match="Triton RMSNorm unavailable"):
        normalized = norm(hidden)
    expected = hidden * torch.rsqrt(hidden.pow(2).mean(dim=-1, keepdim=True) + norm.eps)
    torch.testing.assert_close(normalized, expected * norm.weight)
    assert norm._triton_fallback_warned
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # warn once only
        norm(hidden)

    swiglu = SwiGLU(8, 16, use_triton_swiglu=True)
    with pytest.warns(RuntimeWarning, match="Triton SwiGLU unavailable"):
        fused = swiglu(hidden)
    expected_swiglu = swiglu.down_projection(
        F.silu(swiglu.gate_projection(hidden)) * swiglu.up_projection(hidden)
    )
    torch.testing.assert_close(fused, expected_swiglu)

    query = torch.randn(2, 4, 3, 8)
    key = torch.randn(2, 4, 3, 8)
    fast = RotaryEmbedding(8, use_triton_rope=True)
    native = RotaryEmbedding(8)
    with pytest.warns(RuntimeWarning, match="Triton RoPE unavailable"):
        fq, fk = fast(query, key)
    nq, nk = native(query, key)
    torch.testing.assert_close(fq, nq)
    torch.testing.assert_close(fk, nk)


def test_rope_dot_product_depends_only_on_relative_position():
    torch.manual_seed(0)
    d = 8
    q = torch.randn(1, 1, 1, d).expand(-1, -1, 12, -1).clone()
    k = torch.randn(1, 1, 1, d).expand(-1, -1, 12, -1).clone()
    cos, sin = rotary_cos_sin(12, d, 10_000.0, device=q.device, dtype=q.dtype)
    for apply in (apply_rotary_embedding, apply_rotary_embedding_rotate_half):
        rq, rk = apply(q, cos, sin), apply(k, cos, sin)
        torch.testing.assert_close((rq[:, :, 2] * rk[:, :, 5]).sum(), (rq[:, :, 6] * rk[:, :, 9]).sum())


def test_rotary_embedding_validates_like_reference():
    with pytest.raises(ValueError):
        RotaryEmbedding(7)
    with pytest.raises(ValueError):
        RotaryEmbedding(8, theta=0)
    with pytest.raises(ValueError):
        RotaryEmbedding(8)(torch.randn(2, 4, 3, 8), torch.randn(2, 4, 5, 8))


def test_triton_cross_entropy_cpu_fallback_matches_pytorch():
    logits = torch.tensor([[2.0, 0.0, -1.0], [0.5, 1.5, -0.5]])
    targets = torch.tensor([0, 2], dtype=torch.long)
    ce = CrossEntropyWithFallback(use_triton=True)
    with pytest.warns(RuntimeWarning, match="Triton cross-entropy unavailable"):
        actual = ce(logits, targets)
    torch.testing.assert_close(actual, F.cross_entropy(logits, targets))
    assert abs(actual.item() - 1.2887259920) < 1e-6
    assert callable(triton_cross_entropy)


def test_shifted_cross_entropy_cpu_fallback_is_the_train_loop_expression():
    torch.manual_seed(3)
    logits = torch.randn(2, 5, 7)
    ids = torch.randint(0, 7, (2, 5))
    ids[0, 2] = -100
    ce = CrossEntropyWithFallback(use_triton=True)
    with pytest.warns(RuntimeWarning, match="Triton cross-entropy unavailable"):
        actual = ce(logits, ids, shift=True)
    torch.testing.assert_close(actual, F.cross_entropy(logits[:, :-1, :].transpose(1, 2), ids[:, 1:]))
    plain = CrossEntropyWithFallback(use_triton=False)
    torch.testing.assert_close(plain(logits, ids, shift=True), actual)


def test_rmsnorm_add_and_norm_cpu_fallback():
    torch.manual_seed(5)
    x, r = torch.randn(2, 3, 8), torch.randn(2, 3, 8)
    norm = RMSNorm(8, eps=1e-6, use_triton_rmsnorm=True)
    with pytest.warns(RuntimeWarning, match="Triton RMSNorm unavailable"):
        h, y = norm.add_and_norm(x, r)
    torch.testing.assert_close(h, x + r, rtol=0, atol=0)
    torch.testing.assert_close(y, RMSNorm(8, eps=1e-6)(x + r), rtol=0, atol=0)


def test_compiled_modules_fall_back_like_eager_on_cpu():
    """Under torch.compile the launch gate still rejects CPU tensors, and the modules take
    their PyTorch path in one graph, with the same values as eagerly."""

    torch._dynamo.reset()
    torch.manual_seed(6)
    norm = RMSNorm(16, use_triton_rmsnorm=True)
    mlp = SwiGLU(16, 32, use_triton_swiglu=True)
    x = torch.randn(3, 16)
    with pytest.warns(RuntimeWarning, match="requires GPU tensors"):
        expected = mlp(norm(x))
    model = torch.nn.Sequential(norm, mlp)
    explained = torch._dynamo.explain(model)(x)
    assert explained.graph_break_count == 0
    torch._dynamo.reset()
    torch.testing.assert_close(torch.compile(model, backend="aot_eager")(x), expected)


def test_adamw_clip_fallback_is_clip_grad_norm_then_step():
    torch.manual_seed(4)
    ref_params = [torch.nn.Parameter(torch.randn(5)), torch.nn.Parameter(torch.randn(3, 2))]
    params = [torch.nn.Parameter(p.detach().clone()) for p in ref_params]
    for p, q in zip(ref_params, params):
        p.grad = torch.randn_like(p) * 4
        q.grad = p.grad.clone()
    ref_opt = AdamW(ref_params, lr=0.01, weight_decay=0.1)
    torch.nn.utils.clip_grad_norm_(ref_params, 1.0)
    ref_opt.step()
    stepper = AdamWStepWithFallback(use_triton=True)
    with pytest.warns(RuntimeWarning, match="Triton AdamW unavailable"):
        stepper.step(AdamW(params, lr=0.01, weight_decay=0.1), max_grad_norm=1.0)
    for p, q in zip(ref_params, params):
        torch.testing.assert_close(q, p, rtol=0, atol=0)
        torch.testing.assert_close(q.grad, p.grad, rtol=0, atol=0)


def test_grad_scaler_fallback_is_the_train_loop_fp16_sequence():
    """On CPU the fused GradScaler update refuses and the fallback runs the reference
    sequence (train_loop.py:155-160): unscale_, clip_grad_norm_, step, update."""

    torch.manual_seed(5)
    ref_params = [torch.nn.Parameter(torch.randn(5)), torch.nn.Parameter(torch.randn(3, 2))]
    params = [torch.nn.Parameter(p.detach().clone()) for p in ref_params]
    scalers = [torch.amp.GradScaler("cpu", init_scale=1024.0, growth_interval=1) for _ in range(2)]
    for sc in scalers:
        sc.scale(torch.ones(()))
    ref_opt, opt = AdamW(ref_params, lr=0.01, weight_decay=0.1), AdamW(params, lr=0.01, weight_decay=0.1)
    stepper = AdamWStepWithFallback(use_triton=True)
    for step in range(2):
        for p, q in zip(ref_params, params):
            p.grad = torch.randn_like(p) * 4 * scalers[0].get_scale()
            q.grad = p.grad.clone()
        scalers[0].unscale_(ref_opt)
        torch.nn.utils.clip_grad_norm_(ref_params, 1.0)
        scalers[0].step(ref_opt)
        scalers[0].update()
        if step == 0:
            with pytest.warns(RuntimeWarning, match="Triton AdamW unavailable"):
                stepper.step_with_grad_scaler(scalers[1], opt, 1.0)
        else:  # warned once
            stepper.step_with_grad_scaler(scalers[1], opt, 1.0)
        for p, q in zip(ref_params, params):
            torch.testing.assert_close(q, p, rtol=0, atol=0)
            torch.testing.assert_close(q.grad, p.grad, rtol=0, atol=0)
        assert scalers[1].get_scale() == scalers[0].get_scale() == 1024.0 * 2 ** (step + 1)
    with pytest.raises(RuntimeError, match="not implemented"):
        triton_grad_scaler_step(scalers[1], opt, 1.0)


def test_adamw_rejects_mismatched_resumed_state_before_anything_runs():
    """A resumed state whose moments do not match the parameter (load_state_dict does not
    check shapes) is refused by the fused step before any pointer is taken; the fallback then
    runs torch's step, which reports the mismatch itself."""

    p = torch.nn.Parameter(torch.randn(6))
    p.grad = torch.randn(6)
    opt = AdamW([p], lr=0.01)
    opt.state[p] = {"step": torch.tensor(3.0), "exp_avg": torch.zeros(4), "exp_avg_sq": torch.zeros(6)}
    with pytest.raises(TritonAdamWUnavailable, match="exp_avg does not match"):
        triton_adamw_step(opt)
    stepper = AdamWStepWithFallback(use_triton=True)
    with pytest.warns(RuntimeWarning, match="Triton AdamW unavailable"):
        with pytest.raises(RuntimeError):
            stepper.step(opt)
    opt.state[p] = {"step": torch.tensor(3.0), "exp_avg": torch.zeros(12)[::2], "exp_avg_sq": torch.zeros(6)}
    with pytest.raises(TritonAdamWUnavailable, match="not contiguous"):
        triton_adamw_step(opt)
    opt.state[p] = {"step": 3.0, "exp_avg": torch.zeros(6), "exp_avg_sq": torch.zeros(6)}
    with pytest.raises(TritonAdamWUnavailable, match="one-element tensor"):
        triton_adamw_step(opt)


def test_adamw_fallback_matches_known_single_step_update():
    parameter = torch.nn.Parameter(torch.tensor([1.0]))
    optimizer = AdamW([parameter], lr=0.1, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    parameter.grad = torch.tensor([1.0])
    step = AdamWStepWithFallback(use_triton=True)
    with pytest.warns(RuntimeWarning, match="Triton AdamW unavailable"):
        step.step(optimizer)
    torch.testing.assert_close(parameter.detach(), torch.tensor([0.899]))
    with pytest.raises(RuntimeError, match="not implemented"):
        triton_adamw_step(optimizer)
    # the fallback left torch's own state untouched by the fused path
    assert float(optimizer.state[parameter]["step"]) == 1.0


def test_detect_triton_support_on_cpu():
    report = detect_triton_support()
    assert not report.enabled and not report.available and not report.hardware_compatible
    assert not detect_triton_support(enabled=True).available


def test_banner_rows_on_cpu():
    # the two kernel rows of the run banner (display.py:315-338), from the live state
    off = kernel_status_rows(TritonKernelsConfig())
    assert off[0] == ("Triton kernels", "off")
    assert off[1] == ("Triton status", "rmsnorm=fallback swiglu=fallback rope=fallback "
                      "attention=fallback cross_entropy=fallback adamw=fallback")
    asked = kernel_status_rows(TritonKernelsConfig(rmsnorm=True, adamw=True))
    assert asked[0] == ("Triton kernels", "requested; fallback: rmsnorm, adamw")


def test_kernel_flags_are_strict_bools():
    cfg = TritonKernelsConfig(rmsnorm=True, swiglu=True)
    assert cfg.rmsnorm and cfg.swiglu and not cfg.rope and not cfg.adamw
    with pytest.raises(ConfigValidationError):
        TritonKernelsConfig(rmsnorm=1)  # type: ignore[arg-type]
    with pytest.raises(ConfigValidationError):
        TritonKernelsConfig.from_mapping({"rmsnorm": True, "layernorm": True})
    assert TritonKernelsConfig.from_mapping({"cross_entropy": True}).cross_entropy


def test_oracle_not_imported_by_product():
    import pathlib
    import re

    pkg = pathlib.Path(__file__).resolve().parents[1] / "picotron_amd"
    for path in pkg.rglob("*.py"):
        assert not re.search(r"^\s*(from|import)\s+oracle\b", path.read_text(), flags=re.M), path
