"""The launch-tuning overrides (resident-workgroup limits, read once per process from the
environment) change speed only: two child processes with different limits must produce
bit-identical outputs from the same seeded inputs."""

from __future__ import annotations

import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

_SCRIPT = textwrap.dedent("""
    import hashlib, sys
    sys.path.insert(0, {root!r})
    import torch
    from picotron_amd import ops
    from picotron_amd.nn.triton_kernels import triton_adamw_step

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    def randn(*shape, dtype=torch.bfloat16):
        return torch.randn(shape, generator=gen, device=dev).to(dtype)

    digest = hashlib.sha256()
    def add(*tensors):
        for t in tensors:
            digest.update(t.detach().contiguous().reshape(-1).view(torch.uint8).cpu().numpy().tobytes())

    g, u, dy = randn(3 << 20), randn(3 << 20), randn(3 << 20)
    add(ops.swiglu_fwd(g, u), *ops.swiglu_bwd(dy, g, u))
    x, w, gy = randn(3000, 4096), randn(4096), randn(3000, 4096)
    y, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    add(y, rstd, *ops.rmsnorm_bwd(gy, x, w, rstd))
    q, k = randn(2, 512, 8, 128).transpose(1, 2), randn(2, 512, 2, 128).transpose(1, 2)
    ang = torch.outer(torch.arange(512, device=dev, dtype=torch.float32),
                      1.0 / 5e5 ** (torch.arange(0, 128, 2, device=dev, dtype=torch.float32) / 128))
    add(*ops.rope(q, ang.cos(), ang.sin(), layout="rotate_half", x1=k))
    logits = randn(300, 50257) * 2
    targets = torch.randint(0, 50257, (300,), generator=gen, device=dev)
    loss, ws = ops.cross_entropy(logits, targets, write_grad=True)
    ops.cross_entropy_scale_grad(logits, targets, torch.tensor(0.37, device=dev), workspace=ws)
    add(loss, logits)
    logits16 = (randn(300, 32000) * 2).half()
    loss16, ws16 = ops.cross_entropy(logits16, targets % 32000, write_grad=True)
    ops.cross_entropy_scale_grad(logits16, targets % 32000, torch.tensor(4096.0, device=dev), workspace=ws16)
    add(loss16, logits16)
    p = torch.nn.Parameter(randn(1 << 20, dtype=torch.float32))
    p.grad = randn(1 << 20, dtype=torch.float32)
    opt = torch.optim.AdamW([p], lr=1e-3, weight_decay=0.1)
    triton_adamw_step(opt)
    add(p, opt.state[p]["exp_avg"], opt.state[p]["exp_avg_sq"])
    torch.cuda.synchronize()
    print(digest.hexdigest())
""")

_KNOBS = ("PT_ADAMW_BLOCKS_PER_CU", "PT_SWIGLU_FWD_OCCUPANCY", "PT_SWIGLU_BWD_OCCUPANCY",
          "PT_CE_SCALE_OCCUPANCY", "PT_CE_OCCUPANCY", "PT_ROPE_OCCUPANCY",
          "PT_RMSNORM_FWD_OCCUPANCY", "PT_RMSNORM_BWD_OCCUPANCY", "PT_CE_DEFER_OCCUPANCY",
          "PT_CE_SCALE_BLOCKS_PER_CU")


def _digest(env_values: dict[str, str]) -> str:
    env = {k: v for k, v in os.environ.items() if k not in _KNOBS}
    env.update(env_values)
    root = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-c", _SCRIPT.format(root=root)], env=env,
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return proc.stdout.strip().splitlines()[-1]


def test_occupancy_limits_change_speed_only(gpu):
    unlimited = _digest({k: "0" for k in _KNOBS})
    limited = _digest({k: v for k, v in zip(_KNOBS, ("2", "3", "1", "2", "1", "4", "5", "1", "2", "8"))})
    assert unlimited == limited
