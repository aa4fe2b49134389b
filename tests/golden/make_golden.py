"""Regenerate the golden fixtures in this directory from the (pinned) fp64 oracle.

    python tests/golden/make_golden.py

Inputs are seeded CPU tensors at the reference's quickstart shapes (or small shapes for
the other ops); outputs are the fp64 oracle rounded to fp32.  ``tests/test_golden.py``
re-derives every file and requires an exact match, and the GPU tests compare the HIP
kernels against these files.  Also records the reference's two known-answer tests
(tests/test_triton_ce_adamw.py:15-38 in AndyMLAndAI/picotron).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import adamw as o_adamw  # noqa: E402
from oracle import cross_entropy as o_ce  # noqa: E402
from oracle import rmsnorm as o_rms  # noqa: E402
from oracle import rope as o_rope  # noqa: E402
from oracle import swiglu as o_swiglu  # noqa: E402


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).numpy()


def build() -> dict[str, dict[str, np.ndarray]]:
    out: dict[str, dict[str, np.ndarray]] = {}

    # RMSNorm, quickstart config: x [128 tokens (2x64), 128], w ~ 1 + 0.02 N(0,1), eps 1e-6
    g = torch.Generator().manual_seed(1)
    x = torch.randn(128, 128, generator=g)
    w = 1 + 0.02 * torch.randn(128, generator=g)
    dy = torch.randn(128, 128, generator=g)
    y, rstd = o_rms.forward(x, w, 1e-6)
    dx, dw = o_rms.backward(dy, x, w, 1e-6)
    out["rmsnorm_quickstart"] = dict(
        x=_f32(x), w=_f32(w), dy=_f32(dy), eps=np.float64(1e-6),
        y=_f32(y), rstd=_f32(rstd), dx=_f32(dx), dw=_f32(dw),
    )

    # SwiGLU, quickstart gate/up shape [128, 256] (first 32 rows kept to stay small)
    g = torch.Generator().manual_seed(1)
    gate = torch.randn(128, 256, generator=g)[:32].contiguous()
    up = torch.randn(128, 256, generator=g)[:32].contiguous()
    dyy = torch.randn(32, 256, generator=g)
    dg, du = o_swiglu.backward(dyy, gate, up)
    out["swiglu_quickstart"] = dict(
        gate=_f32(gate), up=_f32(up), dy=_f32(dyy), y=_f32(o_swiglu.forward(gate, up)),
        dgate=_f32(dg), dup=_f32(du),
    )

    # RoPE: (B, H, S, D) = (2, 4, 16, 8), theta 5e5, both layouts, forward and inverse
    g = torch.Generator().manual_seed(4)
    xs = torch.randn(2, 4, 16, 8, generator=g)
    cos, sin = o_rope.tables(16, 8, 500_000.0)
    rope = dict(x=_f32(xs), cos=_f32(cos), sin=_f32(sin))
    for layout in ("interleaved", "rotate_half"):
        rope[f"y_{layout}"] = _f32(o_rope.rotate(xs, cos, sin, layout))
        rope[f"inv_{layout}"] = _f32(o_rope.rotate(xs, cos, sin, layout, inverse=True))
    out["rope_small"] = rope

    # Cross-entropy: logits [16, 1000] ~ N(0, 2^2), 3 ignored targets
    g = torch.Generator().manual_seed(5)
    logits = 2 * torch.randn(16, 1000, generator=g)
    targets = torch.randint(0, 1000, (16,), generator=g)
    targets[[2, 7, 11]] = -100
    loss, grad = o_ce.forward_backward(logits, targets)
    out["cross_entropy_small"] = dict(
        logits=_f32(logits), targets=targets.numpy(), loss=np.float64(loss.item()), grad=_f32(grad)
    )
    kat_logits = torch.tensor([[2.0, 0.0, -1.0], [0.5, 1.5, -0.5]])
    kat_targets = torch.tensor([0, 2])
    kat_loss, kat_grad = o_ce.forward_backward(kat_logits, kat_targets)
    out["cross_entropy_reference_kat"] = dict(
        logits=_f32(kat_logits), targets=kat_targets.numpy(), loss=np.float64(1.2887259920),
        oracle_loss=np.float64(kat_loss.item()), grad=_f32(kat_grad),
    )

    # AdamW: three tensors (4096+1, 17, 1 elements), 3 steps, the cfg hyperparameters
    g = torch.Generator().manual_seed(6)
    sizes = (4097, 17, 1)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    adam: dict[str, np.ndarray] = {"sizes": np.array(sizes), "steps": np.int64(3)}
    for i, n in enumerate(sizes):
        p = 0.02 * torch.randn(n, generator=g, dtype=torch.float64)
        m = torch.zeros(n, dtype=torch.float64)
        v = torch.zeros(n, dtype=torch.float64)
        adam[f"p0_{i}"] = _f32(p)
        p = torch.from_numpy(adam[f"p0_{i}"]).double()
        for t in range(1, 4):
            grad_t = (1e-3 * torch.randn(n, generator=g)).float()
            adam[f"g{t}_{i}"] = _f32(grad_t)
            p, m, v = o_adamw.step(p, grad_t.double(), m, v, t=t, **hp)
        adam[f"p_{i}"], adam[f"m_{i}"], adam[f"v_{i}"] = _f32(p), _f32(m), _f32(v)
    out["adamw_small"] = adam
    one = torch.tensor([1.0], dtype=torch.float64)
    kp, _, _ = o_adamw.step(one, one, 0 * one, 0 * one, t=1, lr=0.1, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)
    out["adamw_reference_kat"] = dict(p=np.float64(0.899), oracle_p=np.float64(kp.item()))
    return out


def main() -> None:
    for name, arrays in build().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
