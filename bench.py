"""Benchmark of the fused memory-bound kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload headline|rmsnorm|residual_rmsnorm|swiglu|rope|ce|ce_train|ce_train_fp16|ce_demo_fp16|ce_vocabs|adamw|adamw_list|adamw_clip|zero_step|fp16_step|modules|copy]

Default workload (the headline metric, "RMSNorm/SwiGLU fwd+bwd"): ``--layers`` decoder layers
(default 4), each with its own activations: the RMSNorm forward of a bf16 [16384 tokens
(8 x 2048), 4096] activation (eps 1e-5, bf16 weight, rstd kept in fp32) and the SwiGLU
forward of bf16 [16384, 14336] gate/up, then the backwards in reverse layer order.  A layer's
working set (3.4 GB) is far above the 256 MB Infinity Cache, so no input is cache-resident
when it is read.  Inputs are synthetic (seeded N(0,1), weight 1 + 0.02 N(0,1)) and resident
in HBM before timing.  The line also carries each op timed alone (``config.ops``: the
per-op GB/s and % of peak the >=75% target is stated for), every kernel's event timing
(``roofline.per_kernel``) and compact figures for the RoPE, cross-entropy and AdamW
configurations (``config.other_configs``).

Prints ONE JSON line: value = algorithmic bytes of the step / wall time of the step
(decimal GB/s) over K timed steps bracketed by device synchronisations, with a
``roofline`` object for the dominant kernel (HIP events around each of its launches, on
the stream they run on, over a second pass of the same K steps -- the event records cost a
few microseconds per launch, so that pass is kept out of the value) and a ``cpu_baseline``
object (the reference's PyTorch fallback, restated in ``oracle/``, timed on this host's
cores on a bounded sample of the same inputs).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch
from torch.nn import functional as F

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from picotron_amd import _lib, ops  # noqa: E402

PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
HEADLINE_METRIC = "RMSNorm/SwiGLU fwd+bwd HBM GB/s & % of peak, 16k tok×4096 bf16"


def _seeded(shape, dtype, seed, scale=1.0, shift=0.0, device="cuda"):
    g = torch.Generator(device=device).manual_seed(seed)
    out = torch.empty(shape, dtype=dtype, device=device)
    # generate in fp32 slices to bound the temporary
    flat = out.view(-1)
    step = 1 << 28
    for lo in range(0, flat.numel(), step):
        hi = min(flat.numel(), lo + step)
        flat[lo:hi] = (torch.randn(hi - lo, generator=g, device=device) * scale + shift).to(dtype)
    return out


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _cpu_info() -> tuple[int, int, str]:
    cores = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return cores, os.cpu_count() or cores, model


CPU_TARGET_S = 10.0  # CPU work per baseline measurement


def _time_cpu(fn, target_s: float = CPU_TARGET_S, setup=None) -> tuple[float, int]:
    """(median seconds per call, calls timed): one warm-up call, then calls until about
    ``target_s`` seconds of CPU work (at least 3).  ``setup`` (untimed) runs before each
    call, e.g. to restore inputs that the call modifies in place."""

    if setup is not None:
        setup()
    fn()
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < target_s and len(times) < 1000):
        if setup is not None:
            setup()
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# ------------------------------------------------------------------ workloads


class Workload:
    name = ""
    metric = ""
    dtype = "bf16"
    description = ""
    dominant = ""
    dominant_bytes = 0
    bytes_per_step = 0
    tokens_per_step = 0
    launches_per_step = 1  # timed launches of the dominant kernel per step (one per layer where layered)

    def step(self, events: list | None) -> None:
        raise NotImplementedError

    def cpu_baseline(self) -> dict:
        raise NotImplementedError

    def extra(self, steps: int) -> dict | None:
        """Additional figures measured after the timed passes (reported under config)."""

        return None


class RMSNormWorkload(Workload):
    name = "rmsnorm"
    metric = HEADLINE_METRIC
    rows, cols, eps = 16384, 4096, 1e-5
    storage = torch.bfloat16  # activations and weight

    def __init__(self, layers: int) -> None:
        self.layers = layers
        self.launches_per_step = layers
        r, c, st = self.rows, self.cols, self.storage
        code = ops.dtype_code(st)
        self.w = _seeded((c,), st, 2, 0.02, 1.0)
        self.x = [_seeded((r, c), st, 10 + i) for i in range(layers)]
        self.dy = [_seeded((r, c), st, 20 + i) for i in range(layers)]
        self.y = [torch.empty_like(t) for t in self.x]
        self.dx = [torch.empty_like(t) for t in self.x]
        self.rstd = [torch.empty(r, dtype=torch.float32, device="cuda") for _ in range(layers)]
        self.dw = [torch.empty(c, dtype=st, device="cuda") for _ in range(layers)]
        lib = _lib.lib()
        self.ws_bytes = lib.pt_rmsnorm_bwd_workspace_bytes(r, c, code)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device="cuda")
        s = sw = torch.tensor([], dtype=st).element_size()
        self.fwd_bytes = 2 * r * c * s + c * sw + 4 * r
        self.bwd_bytes = 3 * r * c * s + 2 * c * sw + 4 * r
        self.bytes_per_step = layers * (self.fwd_bytes + self.bwd_bytes)
        self.tokens_per_step = layers * r
        self.dominant = "rmsnorm backward (rmsnorm_bwd_kernel row pass + rmsnorm_dw_finish_kernel)"
        self.dominant_bytes = self.bwd_bytes
        tname = {torch.bfloat16: "bf16", torch.float32: "fp32"}[st]
        self.description = (
            f"RMSNorm fwd+bwd {tname} [16384 tokens (8x2048), 4096], eps 1e-5, {tname} weight, fp32 rstd; "
            f"step = forward of {layers} independent activations then backward in reverse"
        )
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self._fwd = [
            (lib.pt_rmsnorm_fwd, (_p(self.x[i]), c, _p(self.w), _p(self.y[i]), c, _p(self.rstd[i]),
                                  r, c, ctypes.c_float(self.eps), code, code, stream))
            for i in range(layers)
        ]
        self._bwd = [
            (lib.pt_rmsnorm_bwd, (_p(self.dy[i]), c, _p(self.x[i]), c, _p(self.w), _p(self.rstd[i]),
                                  _p(self.dx[i]), c, _p(self.dw[i]), _p(self.ws), self.ws_bytes, r, c,
                                  code, code, stream))
            for i in range(layers)
        ]

    def step(self, events):
        for fn, args in self._fwd:
            rc = fn(*args)
            if rc:
                _lib.check("pt_rmsnorm_fwd", rc)
        for fn, args in reversed(self._bwd):
            if events is not None:
                start, end = events.pop()
                start.record()
            rc = fn(*args)
            if events is not None:
                end.record()
            if rc:
                _lib.check("pt_rmsnorm_bwd", rc)

    def extra(self, steps: int) -> dict:
        """The forward against a plain copy of the same traffic (one 134 MB stream in, one out,
        over the same rotating per-layer buffers), both timed per launch with HIP events on the
        launch stream: how close the norm comes to data movement alone at this size."""

        lib = _lib.lib()
        nbytes = self.rows * self.cols * 2
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

        def per_launch_us(launch) -> float:
            for i in range(self.layers):
                launch(i)
            pairs = []
            for _ in range(steps):
                for i in range(self.layers):
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    launch(i)
                    b.record()
                    pairs.append((a, b))
            torch.cuda.synchronize()
            return statistics.median(a.elapsed_time(b) * 1e3 for a, b in pairs)

        def fwd(i):
            fn, args = self._fwd[i]
            _lib.check("pt_rmsnorm_fwd", fn(*args))

        def copy(i):
            _lib.check("pt_copy", lib.pt_copy(_p(self.x[i]), _p(self.y[i]), nbytes, stream))

        fwd_us = per_launch_us(fwd)
        copy_us = per_launch_us(copy)
        return {
            "forward_median_launch_us": round(fwd_us, 2),
            "forward_gbs": round(self.fwd_bytes / fwd_us / 1e3, 1),
            "same_size_copy_median_launch_us": round(copy_us, 2),
            "same_size_copy_gbs": round(2 * nbytes / copy_us / 1e3, 1),
        }

    def cpu_baseline(self) -> dict:
        from oracle import rmsnorm as o_rms

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        rows = self.rows
        x, dy, w = self.x[0].cpu(), self.dy[0].cpu(), self.w.cpu()
        sec, calls = _time_cpu(lambda: o_rms.fallback_forward_backward(x, w, self.eps, dy))
        c = self.cols
        s = x.element_size()
        nbytes = 5 * rows * c * s + 3 * c * s + 8 * rows
        return dict(
            value=nbytes / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"one activation [{rows}, {c}] (one of the step's {self.layers} layers): reference PyTorch "
                   f"fallback fwd+bwd (rmsnorm.py:56-60,113-134) on {x.dtype} CPU tensors, median of {calls} "
                   f"calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=rows / sec,
        )


class RMSNormFp32Workload(RMSNormWorkload):
    """RMSNorm at the headline shape in fp32, the storage type the decoder feeds its norms in
    training (picotron_decoder.py:116-123,186: the residual stream stays fp32)."""

    name = "rmsnorm_fp32"
    metric = "RMSNorm fwd+bwd HBM GB/s & % of peak, 16k tok x 4096 fp32"
    dtype = "f32"
    storage = torch.float32


class ResidualRMSNormWorkload(Workload):
    """The decoder block's residual add fused with the norm after it (reference
    src/picotron/models/picotron_decoder.py:116-119), forward and backward."""

    name = "residual_rmsnorm"
    metric = "Residual add + RMSNorm fwd+bwd HBM GB/s & % of peak, 16k tok x 4096 bf16"
    rows, cols, eps = 16384, 4096, 1e-5

    def __init__(self, layers: int) -> None:
        self.layers = layers
        self.launches_per_step = layers
        r, c = self.rows, self.cols
        bf = torch.bfloat16
        self.w = _seeded((c,), bf, 2, 0.02, 1.0)
        self.x = [_seeded((r, c), bf, 30 + i) for i in range(layers)]
        self.res = [_seeded((r, c), bf, 40 + i) for i in range(layers)]
        self.dy = [_seeded((r, c), bf, 50 + i) for i in range(layers)]
        self.dh_in = [_seeded((r, c), bf, 60 + i) for i in range(layers)]
        self.h = [torch.empty_like(t) for t in self.x]
        self.y = [torch.empty_like(t) for t in self.x]
        self.dh = [torch.empty_like(t) for t in self.x]
        self.rstd = [torch.empty(r, dtype=torch.float32, device="cuda") for _ in range(layers)]
        self.dw = [torch.empty(c, dtype=bf, device="cuda") for _ in range(layers)]
        lib = _lib.lib()
        self.lib = lib
        self.ws_bytes = lib.pt_rmsnorm_bwd_workspace_bytes(r, c, _lib.PT_BFLOAT16)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device="cuda")
        s = 2
        self.fwd_bytes = 4 * r * c * s + c * s + 4 * r
        self.bwd_bytes = 4 * r * c * s + 2 * c * s + 4 * r
        self.bytes_per_step = layers * (self.fwd_bytes + self.bwd_bytes)
        self.tokens_per_step = layers * r
        self.dominant = "fused residual + rmsnorm backward (rmsnorm_bwd_kernel with dh_in + rmsnorm_dw_finish_kernel)"
        self.dominant_bytes = self.bwd_bytes
        self.description = (
            f"h = x + residual; y = RMSNorm(h) and its backward dh = norm_bwd(dy) + dh_in, bf16 "
            f"[16384 tokens, 4096], eps 1e-5, bf16 weight; step = forward of {layers} layers then "
            f"backward in reverse"
        )
        self.stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        bfc = _lib.PT_BFLOAT16
        self._fwd = [
            (lib.pt_residual_rmsnorm_fwd, (_p(self.x[i]), c, _p(self.res[i]), c, _p(self.w), _p(self.h[i]), c,
                                           _p(self.y[i]), c, _p(self.rstd[i]), r, c, ctypes.c_float(self.eps),
                                           bfc, bfc, self.stream))
            for i in range(layers)
        ]
        self._bwd = [
            (lib.pt_residual_rmsnorm_bwd, (_p(self.dy[i]), c, _p(self.dh_in[i]), c, _p(self.h[i]), c, _p(self.w),
                                           _p(self.rstd[i]), _p(self.dh[i]), c, _p(self.dw[i]), _p(self.ws),
                                           self.ws_bytes, r, c, bfc, bfc, self.stream))
            for i in range(layers)
        ]

    def step(self, events):
        for fn, args in self._fwd:
            rc = fn(*args)
            if rc:
                _lib.check("pt_residual_rmsnorm_fwd", rc)
        for fn, args in reversed(self._bwd):
            if events is not None:
                start, end = events.pop()
                start.record()
            rc = fn(*args)
            if events is not None:
                end.record()
            if rc:
                _lib.check("pt_residual_rmsnorm_bwd", rc)

    def extra(self, steps: int) -> dict:
        """The same step unfused: torch's add, then the plain norm kernels, then torch's add of
        the two gradients of h."""

        lib, r, c, bfc = self.lib, self.rows, self.cols, _lib.PT_BFLOAT16

        def unfused():
            for i in range(self.layers):
                torch.add(self.x[i], self.res[i], out=self.h[i])
                _lib.check("pt_rmsnorm_fwd", lib.pt_rmsnorm_fwd(
                    _p(self.h[i]), c, _p(self.w), _p(self.y[i]), c, _p(self.rstd[i]), r, c,
                    ctypes.c_float(self.eps), bfc, bfc, self.stream))
            for i in reversed(range(self.layers)):
                _lib.check("pt_rmsnorm_bwd", lib.pt_rmsnorm_bwd(
                    _p(self.dy[i]), c, _p(self.h[i]), c, _p(self.w), _p(self.rstd[i]), _p(self.dh[i]), c,
                    _p(self.dw[i]), _p(self.ws), self.ws_bytes, r, c, bfc, bfc, self.stream))
                self.dh[i].add_(self.dh_in[i])

        unfused()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            unfused()
        torch.cuda.synchronize()
        return {"unfused_add_then_norm_ms_per_step": round((time.perf_counter() - t0) / steps * 1e3, 4)}

    def cpu_baseline(self) -> dict:
        from oracle import rmsnorm as o_rms

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        rows = self.rows
        x, res, w = self.x[0].cpu(), self.res[0].cpu(), self.w.cpu()
        dy, dh_in = self.dy[0].cpu(), self.dh_in[0].cpu()

        def call():
            h = x + res
            o_rms.fallback_forward_backward(h, w, self.eps, dy)[2].add_(dh_in)

        sec, calls = _time_cpu(call)
        c = self.cols
        nbytes = 8 * rows * c * 2 + 3 * c * 2 + 8 * rows
        return dict(
            value=nbytes / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"one layer [{rows}, {c}]: bf16 add, the reference PyTorch RMSNorm fallback fwd+bwd "
                   f"(rmsnorm.py:56-60,113-134) and the add of the two gradients of h, on CPU, median "
                   f"of {calls} calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=rows / sec,
        )


class SwiGLUWorkload(Workload):
    name = "swiglu"
    metric = "SwiGLU fwd+bwd HBM GB/s & % of peak, 16k tok×14336 bf16"
    rows, cols = 16384, 14336

    def __init__(self, layers: int) -> None:
        self.layers = layers
        self.launches_per_step = layers
        n = self.rows * self.cols
        self.n = n
        self.g = [_seeded((n,), torch.bfloat16, 30 + i) for i in range(layers)]
        self.u = [_seeded((n,), torch.bfloat16, 40 + i) for i in range(layers)]
        self.dy = [_seeded((n,), torch.bfloat16, 50 + i) for i in range(layers)]
        self.y = [torch.empty_like(t) for t in self.g]
        self.dg = [torch.empty_like(t) for t in self.g]
        self.du = [torch.empty_like(t) for t in self.g]
        lib = _lib.lib()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.bytes_per_step = layers * 8 * n * 2
        self.tokens_per_step = layers * self.rows
        self.dominant = "swiglu_bwd_kernel"
        self.dominant_bytes = 5 * n * 2
        self.description = (
            f"SwiGLU fwd+bwd bf16 gate/up [16384, 14336]; step = forward of {layers} independent "
            f"activations then backward in reverse"
        )
        self._fwd = [(lib.pt_swiglu_fwd, (_p(self.g[i]), _p(self.u[i]), _p(self.y[i]), n, _lib.PT_BFLOAT16, stream))
                     for i in range(layers)]
        self._bwd = [(lib.pt_swiglu_bwd, (_p(self.dy[i]), _p(self.g[i]), _p(self.u[i]), _p(self.dg[i]),
                                          _p(self.du[i]), n, _lib.PT_BFLOAT16, stream)) for i in range(layers)]

    def step(self, events):
        for fn, args in self._fwd:
            if fn(*args):
                _lib.check("pt_swiglu_fwd", 1)
        for fn, args in reversed(self._bwd):
            if events is not None:
                start, end = events.pop()
                start.record()
            rc = fn(*args)
            if events is not None:
                end.record()
            if rc:
                _lib.check("pt_swiglu_bwd", rc)

    def cpu_baseline(self) -> dict:
        from oracle import swiglu as o_swiglu

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        rows = self.rows
        n = rows * self.cols
        g, u, dy = self.g[0][:n].cpu(), self.u[0][:n].cpu(), self.dy[0][:n].cpu()
        sec, calls = _time_cpu(lambda: o_swiglu.fallback_forward_backward(g, u, dy))
        return dict(
            value=8 * n * 2 / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"one layer [{rows}, {self.cols}]: reference PyTorch fallback fwd+bwd "
                   f"(F.silu*up, swiglu.py:75-81) on bf16 CPU tensors, median of {calls} calls "
                   f"(~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=rows / sec,
        )


class HeadlineWorkload(Workload):
    """The headline pair as consecutive decoder layers run it: per layer the RMSNorm forward of
    a [16384, 4096] bf16 activation, then the SwiGLU forward of [16384, 14336] bf16 gate/up;
    then the backwards in reverse layer order (SwiGLU, then RMSNorm).  Every layer has its own
    activations (each layer's set is 3.4 GB against a 256 MB Infinity Cache), so no input is
    cache-resident when it is read.  Reference paths: src/picotron/nn/triton_kernels/
    rmsnorm.py:87-134 and swiglu.py:56-81, behind picotron_decoder.py:32-46 and
    feedforward.py:26-43."""

    name = "headline"
    metric = HEADLINE_METRIC

    def __init__(self, layers: int) -> None:
        self.layers = layers
        self.rms = RMSNormWorkload(layers)
        self.swiglu = SwiGLUWorkload(layers)
        n = self.swiglu.n
        self.bytes_per_step = self.rms.bytes_per_step + self.swiglu.bytes_per_step
        self.tokens_per_step = layers * RMSNormWorkload.rows
        self.kinds = {
            "rmsnorm_forward": dict(op="rmsnorm", kernel="rmsnorm_fwd_kernel",
                                    bytes=self.rms.fwd_bytes, calls=self.rms._fwd),
            "rmsnorm_backward": dict(op="rmsnorm", kernel="rmsnorm_bwd_kernel + rmsnorm_dw_finish_kernel",
                                     bytes=self.rms.bwd_bytes, calls=self.rms._bwd),
            "swiglu_forward": dict(op="swiglu", kernel="swiglu_fwd_kernel", bytes=3 * n * 2,
                                   calls=self.swiglu._fwd),
            "swiglu_backward": dict(op="swiglu", kernel="swiglu_bwd_kernel", bytes=5 * n * 2,
                                    calls=self.swiglu._bwd),
        }
        self.timed_kinds = {kind: layers for kind in self.kinds}
        self.description = (
            f"RMSNorm fwd+bwd bf16 [16384 tokens (8x2048), 4096] (eps 1e-5, bf16 weight, fp32 rstd) and "
            f"SwiGLU fwd+bwd bf16 gate/up [16384, 14336]; step = {layers} decoder layers: per layer the "
            f"norm forward then the SwiGLU forward, then the backwards in reverse layer order"
        )

    def _launch(self, kind: str, i: int, events) -> None:
        fn, args = self.kinds[kind]["calls"][i]
        if events is not None:
            start, end = events[kind].pop()
            start.record()
        rc = fn(*args)
        if events is not None:
            end.record()
        if rc:
            _lib.check(fn.__name__, rc)

    def step(self, events):
        for i in range(self.layers):
            self._launch("rmsnorm_forward", i, events)
            self._launch("swiglu_forward", i, events)
        for i in reversed(range(self.layers)):
            self._launch("swiglu_backward", i, events)
            self._launch("rmsnorm_backward", i, events)

    def extra(self, steps: int) -> dict:
        """Each op alone over the same buffers (its own fwd+bwd step, host clock: the per-op
        figures the >=75% target is stated for), the norm's forward against a plain copy of
        the same bytes, and compact figures for the other three configurations."""

        ops_out = {}
        for op, wl, shape in (("rmsnorm", self.rms, [16384, 4096]), ("swiglu", self.swiglu, [16384, 14336])):
            sec = _host_time(wl.step, steps)
            gbps = wl.bytes_per_step / sec / 1e9
            ops_out[op] = {
                "shape": shape,
                "layers_per_step": self.layers,
                "algorithmic_bytes_per_step": wl.bytes_per_step,
                "ms_per_step": round(sec * 1e3, 4),
                "us_per_layer_fwd_bwd": round(sec * 1e6 / self.layers, 2),
                "gbs": round(gbps, 1),
                "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
                "tokens_per_s": round(wl.tokens_per_step / sec, 1),
            }
        ops_out["rmsnorm"].update(self.rms.extra(steps))
        # before the other configurations, whose CPU baselines leave the host cores busy
        # for a while, which slows the host-bound eager steps; a failure here (it runs torch's
        # own kernels and graph capture too) is reported in the line rather than ending it
        steps_out = {}
        for key, describe, count in (("quickstart_step", _quickstart_line, 200), ("demo_step", _demo_line, 20)):
            try:
                steps_out[key] = describe(steps=count)
            except Exception as error:  # noqa: BLE001
                steps_out[key] = {"error": f"{type(error).__name__}: {error}"}
        return {"ops": ops_out, "other_configs": _other_configs(steps), **steps_out}

    def cpu_baseline(self) -> dict:
        rms, swiglu = self.rms.cpu_baseline(), self.swiglu.cpu_baseline()
        # value is in GB/s: bytes of one call = value * 1e9 * seconds per call
        nbytes = 1e9 * (rms["value"] * rms["seconds_per_call"] + swiglu["value"] * swiglu["seconds_per_call"])
        sec = rms["seconds_per_call"] + swiglu["seconds_per_call"]
        return dict(
            value=nbytes / sec / 1e9, unit="GB/s", cores=rms["cores"], kind="port",
            sample=f"one layer of each op: RMSNorm [{self.rms.rows}, {self.rms.cols}] and SwiGLU "
                   f"[{self.swiglu.rows}, {self.swiglu.cols}] fwd+bwd through the reference PyTorch fallbacks "
                   f"(rmsnorm.py:56-60,113-134; F.silu*up and swiglu.py:75-81) on bf16 CPU tensors; value = "
                   f"bytes of both / time of both; each the median of ~{CPU_TARGET_S:.0f} s of calls after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=self.rms.rows / sec,
            rmsnorm_gbs=round(rms["value"], 2), swiglu_gbs=round(swiglu["value"], 2),
        )


def _host_time(step, steps: int, warmup: int = 2) -> float:
    """Seconds per call of ``step(None)``: ``warmup`` untimed calls, then ``steps`` calls
    between two device synchronisations."""

    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(None)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


# Whether the secondary lines get their CPU baseline (off with --no-cpu-baseline).
_WITH_CPU_BASELINE = True

OTHER_CONFIGS = ("rope", "ce", "ce_ref_call", "ce_demo_fp16", "adamw", "adamw_list", "rmsnorm_fp32")


def _other_configs(steps: int) -> dict:
    """The other configurations, each built, measured like the headline (host-clock value,
    HIP events per dominant launch, HBM traffic from its committed counter summary, CPU
    baseline on a bounded sample) and freed: RoPE (q [8,2048,32,128] + k [8,2048,8,128],
    rotate-half, 4 layers), the fused cross-entropy ([8192, 128256] bf16, in place), the
    reference's unchanged train-loop call ([4, 2049, 128256] bf16, out of place), the same call
    on the notebook demo's fp16 logits ([32, 256, 50257], loss x 65536), the fused AdamW step (1.2e9 fp32 parameters, as one tensor and as 100) and RMSNorm in fp32, the
    norms' training dtype ([16384, 4096], 4 layers)."""

    out = {}
    for name in OTHER_CONFIGS:
        wl = WORKLOADS[name](DEFAULT_LAYERS[name])
        m = _measure(wl, name, steps, warmup=2)
        sec = m["elapsed"] / steps
        gbps = wl.bytes_per_step / sec / 1e9
        dom = m["per_kernel"][m["dominant"]]
        out[name] = {
            "workload": wl.description,
            "ms_per_step": round(sec * 1e3, 4),
            "gbs": round(gbps, 1),
            "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
            "kernel": dom["kernel"],
            "algorithmic_bytes_per_launch": dom["algorithmic_bytes_per_launch"],
            "avg_launch_us": dom["avg_launch_us"],
            "achieved": dom["achieved"],
            "frac": dom["frac"],
            "traffic": dom["traffic"],
            "traffic_source": m["traffic_source"],
            "cpu_baseline": _cpu_line(wl) if _WITH_CPU_BASELINE else None,
        }
        del wl
        torch.cuda.empty_cache()
    return out


class RoPEWorkload(Workload):
    name = "rope"
    metric = "RoPE fwd+bwd HBM GB/s & % of peak, q[8,2048,32,128] k[8,2048,8,128] bf16"

    def __init__(self, layers: int, layout: str = "rotate_half") -> None:
        from picotron_amd.nn.rope import rotary_cos_sin

        self.layers = layers
        self.launches_per_step = layers
        self.layout = layout
        b, s, hq, hk, d = 8, 2048, 32, 8, 128
        self.cos, self.sin = rotary_cos_sin(s, d, 500_000.0, device=torch.device("cuda"), dtype=torch.float32)
        self.q = [_seeded((b, s, hq, d), torch.bfloat16, 60 + i).transpose(1, 2) for i in range(layers)]
        self.k = [_seeded((b, s, hk, d), torch.bfloat16, 70 + i).transpose(1, 2) for i in range(layers)]
        self.dq = [_seeded((b, s, hq, d), torch.bfloat16, 80 + i).transpose(1, 2) for i in range(layers)]
        self.dk = [_seeded((b, s, hk, d), torch.bfloat16, 90 + i).transpose(1, 2) for i in range(layers)]
        self.yq = [torch.empty_like(t) for t in self.q]
        self.yk = [torch.empty_like(t) for t in self.k]
        self.gq = [torch.empty_like(t) for t in self.q]
        self.gk = [torch.empty_like(t) for t in self.k]
        lib = _lib.lib()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        qk_bytes = (b * s * hq * d + b * s * hk * d) * 2
        self.bytes_per_step = layers * 4 * qk_bytes
        self.tokens_per_step = layers * b * s
        self.dominant = "rope_kernel (query + key forward, one launch)"
        self.dominant_bytes = 2 * qk_bytes
        self.description = (
            f"RoPE fwd+bwd bf16 q [8,2048,32,128], k [8,2048,8,128] in (B,S,H,D) memory, {layout}, "
            f"theta 5e5, fp32 cos/sin; step = forward of {layers} layers then backward in reverse"
        )
        lay = ops.LAYOUTS[layout]
        self._keep = []

        def call(x0, y0, x1, y1, inverse):
            d0, d1 = ops._rope_desc(x0, y0), ops._rope_desc(x1, y1)
            self._keep.extend([d0, d1])
            return (lib.pt_rope, (_p(x0), _p(y0), d0, _p(x1), _p(y1), d1, d, _p(self.cos), _p(self.sin),
                                  s, lay, inverse, _lib.PT_BFLOAT16, stream))

        self._fwd = [call(self.q[i], self.yq[i], self.k[i], self.yk[i], 0) for i in range(layers)]
        self._bwd = [call(self.dq[i], self.gq[i], self.dk[i], self.gk[i], 1) for i in range(layers)]

    def step(self, events):
        for fn, args in self._fwd:
            if events is not None:
                start, end = events.pop()
                start.record()
            rc = fn(*args)
            if events is not None:
                end.record()
            if rc:
                _lib.check("pt_rope", rc)
        for fn, args in reversed(self._bwd):
            rc = fn(*args)
            if rc:
                _lib.check("pt_rope", rc)

    def cpu_baseline(self) -> dict:
        from oracle import rope as o_rope

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        bsz = 8
        q = self.q[0][:bsz].cpu()
        dq = self.dq[0][:bsz].cpu()
        cos, sin = self.cos.cpu().bfloat16(), self.sin.cpu().bfloat16()
        sec, calls = _time_cpu(lambda: o_rope.fallback_forward_backward(q, cos, sin, dq))
        nbytes = 4 * q.numel() * 2
        return dict(
            value=nbytes / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"the query [{bsz}, 32, 2048, 128] of one layer (k excluded): reference eager apply_rotary_embedding "
                   f"(rope.py:35-51, interleaved, bf16 tables) fwd + autograd bwd on CPU, median of {calls} "
                   f"calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=bsz * 2048 / sec,
        )


class CrossEntropyWorkload(Workload):
    name = "ce"
    metric = "Fused cross-entropy fwd+bwd HBM GB/s & % of peak, [8192, 128256] bf16"
    rows, vocab = 8192, 128256

    def __init__(self, layers: int) -> None:
        self.layers = 1
        r, v = self.rows, self.vocab
        self.logits = _seeded((r, v), torch.bfloat16, 100, 2.0)
        g = torch.Generator(device="cuda").manual_seed(101)
        self.targets = torch.randint(0, v, (r,), generator=g, device="cuda")
        self.targets[torch.randperm(r, generator=g, device="cuda")[:410]] = -100
        lib = _lib.lib()
        self.ws_bytes = lib.pt_cross_entropy_workspace_bytes(r)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device="cuda")
        self.loss = torch.empty((), dtype=torch.float32, device="cuda")
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.bytes_per_step = 2 * r * v * 2 + 16 * r
        self.tokens_per_step = r
        self.dominant = "cross-entropy fused fwd+bwd (ce_prepare_kernel + ce_rows_kernel + ce_finish_kernel)"
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "fused cross-entropy fwd+bwd bf16 logits [8192, 128256] ~N(0,2^2), 410 targets = -100, "
            "fp32 mean loss, dlogits written in place; step = one fused call (each step re-reads the "
            "previous step's in-place output as its logits)"
        )
        self._call = (lib.pt_cross_entropy, (_p(self.logits), r, 1, v, 0, v, _p(self.targets), 1, 0, -100,
                                             _p(self.loss), 1, None, 0, 0, _p(self.ws), self.ws_bytes,
                                             _lib.PT_BFLOAT16, stream))

    def step(self, events):
        fn, args = self._call
        if events is not None:
            start, end = events.pop()
            start.record()
        rc = fn(*args)
        if events is not None:
            end.record()
        if rc:
            _lib.check("pt_cross_entropy", rc)

    def cpu_baseline(self) -> dict:
        from oracle import cross_entropy as o_ce

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        rows = 1024
        logits = _seeded((rows, self.vocab), torch.bfloat16, 100, 2.0).cpu()
        targets = self.targets[:rows].cpu()
        sec, calls = _time_cpu(lambda: o_ce.fallback_forward_backward(logits, targets))
        return dict(
            value=(2 * rows * self.vocab * 2 + 16 * rows) / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"{rows} of 8192 rows: F.cross_entropy fwd + autograd bwd on the fp32 upcast (the "
                   f"reference fallback under autocast), median of {calls} calls (~{CPU_TARGET_S:.0f} s) "
                   f"after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=rows / sec,
        )


class CrossEntropyTrainWorkload(Workload):
    """The train loop's loss and its backward through autograd on the model's whole
    (B, S, V) logits, with the shift inside the kernel (reference call:
    src/picotron/training/train_loop.py:141-144)."""

    name = "ce_train"
    metric = "Next-token cross-entropy fwd + autograd bwd HBM GB/s & % of peak, logits [4, 2049, 128256] bf16"
    b, s, vocab = 4, 2049, 128256

    def __init__(self, layers: int) -> None:
        from picotron_amd.nn.triton_kernels import triton_cross_entropy

        self.layers = 1
        b, s, v = self.b, self.s, self.vocab
        self.fn = triton_cross_entropy
        self.leaf = _seeded((b, s, v), torch.bfloat16, 110, 2.0).requires_grad_(True)
        g = torch.Generator(device="cuda").manual_seed(111)
        self.ids = torch.randint(0, v, (b, s), generator=g, device="cuda")
        flat = self.ids[:, 1:].reshape(-1)
        flat[torch.randperm(flat.numel(), generator=g, device="cuda")[: flat.numel() // 20]] = -100
        self.ids[:, 1:] = flat.view(b, s - 1)
        rows = b * s
        self.bytes_per_step = 2 * rows * v * 2 + 16 * rows
        self.tokens_per_step = b * (s - 1)
        self.dominant = ("shifted cross-entropy forward + autograd backward (ce_prepare_kernel + ce_rows_kernel "
                         "+ ce_finish_kernel; the backward's ce_scale_kernel returns at once for grad 1)")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            f"train-loop loss on model logits [{b}, {s}, {v}] bf16 ~N(0,2^2) against input_ids[:, 1:] "
            f"(5% = -100): triton_cross_entropy(logits, input_ids, shift=True) then torch.autograd.grad "
            f"to the logits' leaf; the gradient is written into the logits buffer"
        )

    def _step(self, shifted: bool):
        logits = self.leaf.view(self.b, self.s, self.vocab)
        if shifted:
            loss = self.fn(logits, self.ids, shift=True)
        else:
            loss = self.fn(logits[:, :-1, :].transpose(1, 2), self.ids[:, 1:])
        # to the leaf: the view's backward is a reshape (the logits themselves are a view,
        # whose autograd node is regenerated once the in-place gradient bumps its version)
        (grad,) = torch.autograd.grad(loss, self.leaf)
        return grad

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        self._step(True)
        if events is not None:
            end.record()

    def extra(self, steps: int) -> dict:
        """The same loss through the reference's call shape (sliced, transposed view), whose
        backward adds autograd's slice backward: a zero-filled full-size gradient plus a copy;
        and the reference's own call, F.cross_entropy under bf16 autocast, on the same logits."""

        for _ in range(2):
            self._step(False)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            self._step(False)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / steps * 1e3
        leaf = self.leaf.detach().clone().requires_grad_(True)

        def reference(_events=None):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = torch.nn.functional.cross_entropy(
                    leaf.view(self.b, self.s, self.vocab)[:, :-1, :].transpose(1, 2), self.ids[:, 1:])
            torch.autograd.grad(loss, leaf)

        ref_ms = _host_time(reference, min(steps, 5), warmup=1) * 1e3
        del leaf
        torch.cuda.empty_cache()
        return {"sliced_view_call_ms_per_step": round(ms, 4),
                "torch_autocast_bf16_ms_per_step": round(ref_ms, 4)}

    def cpu_baseline(self) -> dict:
        from oracle import cross_entropy as o_ce

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        s = 257
        logits = self.leaf.detach()[:, :s].cpu()
        ids = self.ids[:, :s].cpu()
        sec, calls = _time_cpu(lambda: o_ce.fallback_forward_backward(
            logits[:, :-1, :].transpose(1, 2), ids[:, 1:]))
        rows = self.b * s
        return dict(
            value=(2 * rows * self.vocab * 2 + 16 * rows) / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"first {s} positions of each sequence: F.cross_entropy fwd + autograd bwd on the fp32 "
                   f"upcast of the sliced view (the reference fallback under autocast), median of {calls} "
                   f"calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=self.b * (s - 1) / sec,
        )


class CrossEntropyReferenceCallWorkload(CrossEntropyTrainWorkload):
    """The train loop's loss call exactly as the reference writes it (train_loop.py:95-97,
    141-144): ``CrossEntropyWithFallback(use_triton=True)`` (drop-in default: the logits are
    left untouched) on ``logits[:, :-1, :].transpose(1, 2)`` against ``input_ids[:, 1:]``, then
    the backward.  The kernel reads the logits and writes the gradient into a new buffer; the
    view is computed on its base, so autograd runs no slice backward."""

    name = "ce_ref_call"
    metric = ("Next-token cross-entropy fwd + autograd bwd through the reference's call site, "
              "HBM GB/s & % of peak, logits [4, 2049, 128256] bf16")

    def __init__(self, layers: int) -> None:
        from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback

        super().__init__(layers)
        self.loss_function = CrossEntropyWithFallback(use_triton=True)
        b, s, v = self.b, self.s, self.vocab
        self.dominant = ("cross-entropy of the reference's call: logits read, gradient written to a new "
                         "buffer (ce_prepare_kernel + ce_rows_kernel + ce_finish_kernel; the backward's "
                         "ce_scale_kernel returns at once for grad 1)")
        self.description = (
            f"the reference's train-loop call on model logits [{b}, {s}, {v}] bf16 ~N(0,2^2): "
            f"CrossEntropyWithFallback(use_triton=True)(logits[:, :-1, :].transpose(1, 2), input_ids[:, 1:]) "
            f"(5% = -100) then torch.autograd.grad to the logits' leaf; the logits are left untouched and "
            f"the gradient goes to a new buffer"
        )

    def _step(self, shifted: bool):
        logits = self.leaf.view(self.b, self.s, self.vocab)
        loss = self.loss_function(logits[:, :-1, :].transpose(1, 2), self.ids[:, 1:])
        (grad,) = torch.autograd.grad(loss, self.leaf)
        return grad

    def extra(self, steps: int) -> dict | None:
        return None


class CrossEntropyTrainFp16Workload(CrossEntropyTrainWorkload):
    """The train loop's loss under fp16 autocast with a GradScaler (reference
    src/picotron/training/train_loop.py:141-144,155-160): fp16 logits, the loss scaled by 65536
    before its backward.  The fp16 forward reads the logits and keeps each row's log-sum-exp; the
    backward reads them again and writes the gradient with the scale applied, rounded once."""

    name = "ce_train_fp16"
    metric = ("Next-token cross-entropy fwd + autograd bwd (fp16, loss scale 65536) HBM GB/s & % of peak, "
              "logits [4, 2049, 128256]")
    dtype = "f16"
    loss_scale = 65536.0

    def __init__(self, layers: int) -> None:
        super().__init__(layers)
        b, s, v = self.b, self.s, self.vocab
        self.leaf = self.leaf.detach().half().requires_grad_(True)
        rows = b * s
        self.bytes_per_step = 3 * rows * v * 2 + 16 * rows  # forward: read; backward: read + write
        self.dominant = ("shifted cross-entropy fp16 forward + autograd backward (ce_prepare_kernel + "
                         "ce_lse_kernel + ce_finish_kernel, then ce_scale_kernel writing the gradient)")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            f"train-loop loss on fp16 model logits [{b}, {s}, {v}] ~N(0,2^2) against input_ids[:, 1:] "
            f"(5% = -100), loss x 65536 (a GradScaler's scale) before torch.autograd.grad to the logits' "
            f"leaf; the forward reads the logits once, the backward reads them and writes the gradient"
        )

    def _step(self, shifted: bool):
        logits = self.leaf.view(self.b, self.s, self.vocab)
        if shifted:
            loss = self.fn(logits, self.ids, shift=True)
        else:
            loss = self.fn(logits[:, :-1, :].transpose(1, 2), self.ids[:, 1:])
        (grad,) = torch.autograd.grad(loss * self.loss_scale, self.leaf)
        return grad

    def extra(self, steps: int) -> dict:
        """The reference's call under fp16 autocast (F.cross_entropy upcasts to fp32) on the same
        logits, its backward with the same scale."""

        leaf = self.leaf.detach().clone().requires_grad_(True)
        ids = self.ids

        def reference(_events=None):
            with torch.autocast("cuda", dtype=torch.float16):
                loss = torch.nn.functional.cross_entropy(
                    leaf.view(self.b, self.s, self.vocab)[:, :-1, :].transpose(1, 2), ids[:, 1:])
            torch.autograd.grad(loss * self.loss_scale, leaf)

        sec = _host_time(reference, min(steps, 5), warmup=1)
        del leaf
        torch.cuda.empty_cache()
        return {"torch_autocast_fp16_ms_per_step": round(sec * 1e3, 4)}

    def cpu_baseline(self) -> dict:
        from oracle import cross_entropy as o_ce

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        s = 257
        logits = self.leaf.detach()[:, :s].cpu()
        ids = self.ids[:, :s].cpu()
        sec, calls = _time_cpu(lambda: o_ce.fallback_forward_backward(
            logits[:, :-1, :].transpose(1, 2), ids[:, 1:]))
        rows = self.b * s
        return dict(
            value=(3 * rows * self.vocab * 2 + 16 * rows) / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"first {s} positions of each sequence, fp16 logits: F.cross_entropy fwd + autograd bwd on "
                   f"the fp32 upcast of the sliced view (the reference fallback under fp16 autocast), median "
                   f"of {calls} calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=self.b * (s - 1) / sec,
        )


class CrossEntropyDemoFp16Workload(CrossEntropyTrainFp16Workload):
    """The notebook demo's loss (examples/kaggle_demo_pretrain_sft_dpo.ipynb, cell 4: GPT-2's
    50257-token vocabulary, micro-batch 32 x sequence 256, fp16 with the train loop's
    GradScaler) through the reference's call site (train_loop.py:95-97,141-144):
    ``CrossEntropyWithFallback(use_triton=True)`` on ``logits[:, :-1, :].transpose(1, 2)``
    against ``input_ids[:, 1:]``, the loss scaled by 65536 before its backward.  A row of 50257
    fp16 logits is 100514 bytes, so rows start on no common 16-byte or 128-byte boundary: the
    kernels split each row at its first 128-byte line."""

    name = "ce_demo_fp16"
    metric = ("Next-token cross-entropy fwd + autograd bwd through the reference's call site (fp16, loss "
              "scale 65536) HBM GB/s & % of peak, logits [32, 256, 50257]")
    b, s, vocab = 32, 256, 50257

    def __init__(self, layers: int) -> None:
        from picotron_amd.nn.triton_kernels import CrossEntropyWithFallback

        super().__init__(layers)
        b, s, v = self.b, self.s, self.vocab
        self.loss_function = CrossEntropyWithFallback(use_triton=True)
        g = torch.Generator(device="cuda").manual_seed(112)
        self.ids = torch.randint(0, v, (b, s), generator=g, device="cuda")  # pretraining: every target kept
        # forward: the b * (s - 1) rows read; backward: read again, the gradient of all b * s
        # rows written (the last position's rows as zeros)
        self.bytes_per_step = (2 * b * (s - 1) + b * s) * v * 2 + 16 * b * s
        self.tokens_per_step = b * (s - 1)
        self.dominant = ("cross-entropy of the reference's call, fp16: ce_prepare_kernel + ce_lse_kernel + "
                         "ce_finish_kernel, then ce_scale_kernel writing the scaled gradient to a new buffer")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            f"the reference's train-loop call on fp16 model logits [{b}, {s}, {v}] ~N(0,2^2): "
            f"CrossEntropyWithFallback(use_triton=True)(logits[:, :-1, :].transpose(1, 2), input_ids[:, 1:]), "
            f"loss x 65536 (a GradScaler's scale) before torch.autograd.grad to the logits' leaf; the logits are "
            f"left untouched and the gradient goes to a new buffer"
        )

    def _step(self, shifted: bool):
        logits = self.leaf.view(self.b, self.s, self.vocab)
        loss = self.loss_function(logits[:, :-1, :].transpose(1, 2), self.ids[:, 1:])
        (grad,) = torch.autograd.grad(loss * self.loss_scale, self.leaf)
        return grad

    def cpu_baseline(self) -> dict:
        from oracle import cross_entropy as o_ce

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        nb = 4
        logits = self.leaf.detach()[:nb].cpu()
        ids = self.ids[:nb].cpu()
        sec, calls = _time_cpu(lambda: o_ce.fallback_forward_backward(
            logits[:, :-1, :].transpose(1, 2), ids[:, 1:]))
        return dict(
            value=((2 * nb * (self.s - 1) + nb * self.s) * self.vocab * 2 + 16 * nb * self.s) / sec / 1e9,
            unit="GB/s", cores=cores, kind="port",
            sample=f"first {nb} of the {self.b} sequences, fp16 logits: F.cross_entropy fwd + autograd bwd on "
                   f"the fp32 upcast of the sliced view (the reference fallback under fp16 autocast), median "
                   f"of {calls} calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, tokens_per_s=nb * (self.s - 1) / sec,
        )


class AdamWWorkload(Workload):
    name = "adamw"
    metric = "Fused AdamW step HBM GB/s & % of peak, 1.2e9 fp32 params"
    dtype = "f32"
    n = 1_200_000_000

    def __init__(self, layers: int) -> None:
        self.layers = 1
        n = self.n
        self.p = _seeded((n,), torch.float32, 110, 0.02)
        self.g = _seeded((n,), torch.float32, 111, 1e-3)
        # the moments as the fused optimizer creates them (ops.adamw_moments: one allocation)
        ((self.m, self.v),) = ops.adamw_moments([self.p])
        host, blocks = ops.adamw_table([self.p], [self.g], [self.m], [self.v])
        self.table = host.cuda()
        self.blocks = blocks
        self.t = 1
        self.bytes_per_step = 28 * n
        self.tokens_per_step = n
        self.dominant = "adamw_kernel"
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "fused AdamW over one flat 1.2e9-element fp32 parameter (p, grad, exp_avg, exp_avg_sq; the "
            "moments in one allocation, as the fused optimizer creates them), lr 3e-4, betas (0.9, 0.95), "
            "eps 1e-8, wd 0.1; step = one optimizer step"
        )
        self.lib = _lib.lib()
        self.stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        rc = self.lib.pt_adamw_step(_p(self.table), 1, self.blocks, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                                    float(self.t), self.stream)
        if events is not None:
            end.record()
        self.t += 1
        if rc:
            _lib.check("pt_adamw_step", rc)

    def cpu_baseline(self) -> dict:
        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        n = 120_000_000
        p = torch.nn.Parameter(self.p[:n].cpu())
        p.grad = self.g[:n].cpu()
        opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
        sec, calls = _time_cpu(opt.step)
        return dict(
            value=28 * n / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"{n:.1e} of 1.2e9 params (1/10): torch.optim.AdamW(foreach=False).step() (the reference "
                   f"fallback, adamw.py:47) on CPU, median of {calls} calls (~{CPU_TARGET_S:.0f} s) after "
                   f"1 warm-up",
            seconds_per_call=sec, params_per_s=n / sec,
        )


class AdamWListWorkload(Workload):
    """The fused AdamW step over a list of 100 fp32 parameters (1.2e9 elements in all), as a
    model's parameter list reaches torch.optim.AdamW (reference src/picotron/training/
    train_loop.py:308-325): the sizes of a decoder stack's projections (16.8M, 4.2M, 58.7M-class
    matrices) with ten 4096-element norm weights among them, each parameter and gradient its own
    allocation, the moments in one as the fused optimizer creates them, one launch for all."""

    name = "adamw_list"
    metric = "Fused AdamW step HBM GB/s & % of peak, 100 fp32 tensors, 1.2e9 params"
    dtype = "f32"

    # per group: four attention projections (16.8M, 4.2M, 4.2M, 16.8M elements), three MLP
    # projections (25.2M), two 1M-element tensors and one 4096-element norm weight
    GROUP = [16_777_216, 4_194_304, 4_194_304, 16_777_216, 25_165_824, 25_165_824, 25_165_824,
             1_048_576, 1_048_576, 4096]

    def __init__(self, layers: int) -> None:
        self.layers = 1
        sizes = self.GROUP * 10
        # pad the last matrix so the total is exactly 1.2e9 elements (a multiple of 1024 keeps
        # every tensor a whole number of 16-byte vectors)
        sizes[-2] += 1_200_000_000 - sum(sizes)
        assert sum(sizes) == 1_200_000_000 and len(sizes) == 100
        self.sizes = sizes
        self.n = sum(sizes)
        self.p = [_seeded((k,), torch.float32, 200 + i, 0.02) for i, k in enumerate(sizes)]
        self.g = [_seeded((k,), torch.float32, 400 + i, 1e-3) for i, k in enumerate(sizes)]
        # the moments as the fused optimizer creates them (ops.adamw_moments: one allocation)
        moments = ops.adamw_moments(self.p)
        self.m = [m for m, _ in moments]
        self.v = [v for _, v in moments]
        host, blocks = ops.adamw_table(self.p, self.g, self.m, self.v)
        self.table = host.cuda()
        self.blocks = blocks
        self.t = 1
        self.bytes_per_step = 28 * self.n
        self.tokens_per_step = self.n
        self.dominant = "adamw_kernel (100 tensors, one launch)"
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "fused AdamW over 100 fp32 parameters of decoder-projection sizes (1.2e9 elements, ten "
            "4096-element norm weights among them), each parameter and gradient its own allocation, the "
            "moments in one (as the fused optimizer creates them), lr 3e-4, betas (0.9, 0.95), "
            "eps 1e-8, wd 0.1; step = one optimizer step (one launch)"
        )
        self.lib = _lib.lib()
        self.stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        rc = self.lib.pt_adamw_step(_p(self.table), len(self.sizes), self.blocks, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                                    float(self.t), self.stream)
        if events is not None:
            end.record()
        self.t += 1
        if rc:
            _lib.check("pt_adamw_step", rc)

    def cpu_baseline(self) -> dict:
        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        params = []
        for p, g in zip(self.p[:10], self.g[:10]):
            q = torch.nn.Parameter(p.cpu())
            q.grad = g.cpu()
            params.append(q)
        n = sum(q.numel() for q in params)
        opt = torch.optim.AdamW(params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
        sec, calls = _time_cpu(opt.step)
        return dict(
            value=28 * n / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"the first 10 of the 100 tensors ({n:.2e} params, one group of sizes): "
                   f"torch.optim.AdamW(foreach=False).step() on CPU, median of {calls} calls "
                   f"(~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, params_per_s=n / sec,
        )


class AdamWClipWorkload(AdamWWorkload):
    """Gradient clipping fused into the AdamW step (the train loop's
    clip_grad_norm_ + step, src/picotron/training/train_loop.py:163-168,338-350)."""

    name = "adamw_clip"
    metric = "Fused grad-norm clip + AdamW step HBM GB/s & % of peak, 1.2e9 fp32 params"

    def __init__(self, layers: int) -> None:
        super().__init__(layers)
        n = self.n
        self.ws_bytes = self.lib.pt_clip_grad_norm_workspace_bytes(self.blocks)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device="cuda")
        self.out = torch.empty(2, dtype=torch.float32, device="cuda")
        self.bytes_per_step = 36 * n  # norm: read g; step: read p, g, m, v, write p, m, v, g
        self.dominant = ("fused clip + step (grad_stats_kernel + grad_stats_finish_kernel + "
                         "adamw_kernel with the clip coefficient, clipped grads written back)")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "torch.nn.utils.clip_grad_norm_(max_norm 1.0) + AdamW step fused, one flat 1.2e9-element "
            "fp32 parameter, lr 3e-4, betas (0.9, 0.95), eps 1e-8, wd 0.1; step = norm pass + one "
            "optimizer pass that scales each gradient by the device-side clip coefficient and writes "
            "it back"
        )

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        out = self.out.data_ptr()
        rc = self.lib.pt_clip_grad_norm(_p(self.table), 1, self.blocks, 1.0, ctypes.c_void_p(out),
                                        ctypes.c_void_p(out + 4), _p(self.ws), self.ws_bytes, self.stream)
        if rc == 0:
            rc = self.lib.pt_adamw_step_scaled(_p(self.table), 1, self.blocks, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                                               float(self.t), ctypes.c_void_p(out + 4), 1, self.stream)
        if events is not None:
            end.record()
        self.t += 1
        if rc:
            _lib.check("pt_clip_grad_norm / pt_adamw_step_scaled", rc)

    def extra(self, steps: int) -> dict:
        """The unfused sequence for comparison: torch's clip_grad_norm_ (foreach norm + scale
        pass) followed by the plain fused step."""

        prm = torch.nn.Parameter(self.p)
        prm.grad = self.g
        def unfused():
            torch.nn.utils.clip_grad_norm_([prm], 1.0)
            rc = self.lib.pt_adamw_step(_p(self.table), 1, self.blocks, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                                        float(self.t), self.stream)
            self.t += 1
            if rc:
                _lib.check("pt_adamw_step", rc)
        unfused()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            unfused()
        torch.cuda.synchronize()
        return {"unfused_clip_then_step_ms_per_step": round((time.perf_counter() - t0) / steps * 1e3, 4)}

    def cpu_baseline(self) -> dict:
        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        n = 120_000_000
        p = torch.nn.Parameter(self.p[:n].cpu())
        g = self.g[:n].cpu()
        opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)

        p.grad = g.clone()

        def clip_step():
            torch.nn.utils.clip_grad_norm_([p], 1.0)
            opt.step()

        sec, calls = _time_cpu(clip_step, setup=lambda: p.grad.copy_(g))
        return dict(
            value=36 * n / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"{n:.1e} of 1.2e9 params (1/10): torch.nn.utils.clip_grad_norm_ + "
                   f"torch.optim.AdamW(foreach=False).step() on CPU (the reference train loop's "
                   f"fallback), median of {calls} calls (~{CPU_TARGET_S:.0f} s) after 1 warm-up",
            seconds_per_call=sec, params_per_s=n / sec,
        )


class ZeroMixedPrecisionStepWorkload(AdamWWorkload):
    """The ZeRO mixed-precision update on one rank (reference src/picotron/parallel/zero.py:
    DistributedGradScaler.step :50-79 -> unscale_and_check_ :139-163 -> clip_grad_norm_
    :165-186 -> the inner AdamW step), fused."""

    name = "zero_step"
    metric = "Fused unscale + inf-check + clip + AdamW step HBM GB/s & % of peak, 1.2e9 fp32 params"
    # Every step unscales the gradients in place and the next step reads them again, so a
    # training-size scale (65536) would shrink them to zero within ten steps, and streams of
    # zeros move about 2 % faster than streams of random data.  With scale 1 the gradients
    # keep their magnitude from step to step; the kernels do the same work for every scale.
    loss_scale = 1.0

    def __init__(self, layers: int) -> None:
        super().__init__(layers)
        from picotron_amd.nn.triton_kernels import triton_unscale_clip_and_step

        n = self.n
        self.fn = triton_unscale_clip_and_step
        self.g.mul_(self.loss_scale)  # gradients as the scaled loss's backward leaves them
        self.g_scaled = self.g.clone()
        self.prm = torch.nn.Parameter(self.p)
        self.prm.grad = self.g
        self.opt = torch.optim.AdamW([self.prm], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
        self.bytes_per_step = 36 * n  # stats: read g; step: read p, g, m, v, write p, m, v, g
        self.dominant = ("fused unscale + clip + step (grad_stats_kernel + grad_stats_finish_kernel, one "
                         "host read of the overflow flag, adamw_kernel with the combined multiplier)")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "ZeRO-1 mixed-precision update on one rank: loss scale 1 (the written-back gradients keep "
            "their magnitude from step to step), finite check, unscale, "
            "clip_grad_norm_(1.0) with the ZeRO rule (scale only if coef < 1) and the AdamW step, one "
            "flat 1.2e9-element fp32 parameter; step = triton_unscale_clip_and_step (each step "
            "unscales and clips the gradients the previous one left)"
        )

    def _rescale(self):
        self.g.copy_(self.g_scaled)

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        found = self.fn(self.opt, self.loss_scale, 1.0)
        if events is not None:
            end.record()
        if found:
            raise RuntimeError("unexpected overflow in the synthetic gradients")

    def extra(self, steps: int) -> dict:
        """The reference sequence on the same data: per-parameter finite check (host sync),
        g *= 1/scale, squared norm (host sync on the coefficient), g *= coef, then the fused
        step (torch's own AdamW step is slower still)."""

        def reference():
            self._rescale()
            g = self.prm.grad
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            if not bool(torch.isfinite(g).all()):
                raise RuntimeError("unexpected overflow")
            g.mul_(1.0 / self.loss_scale)
            sq = torch.zeros((), device=g.device, dtype=torch.float32)
            sq.add_(g.float().pow(2).sum())
            coef = 1.0 / (sq.sqrt() + 1e-6)
            if coef < 1:
                g.mul_(coef.to(dtype=g.dtype))
            from picotron_amd.nn.triton_kernels import triton_adamw_step
            triton_adamw_step(self.opt)
            torch.cuda.synchronize()
            return time.perf_counter() - t0

        reference()
        total = sum(reference() for _ in range(steps))
        return {"reference_sequence_ms_per_step": round(total / steps * 1e3, 4)}

    def cpu_baseline(self) -> dict:
        """The reference ZeRO sequence on one rank (zero.py:139-186, then the inner AdamW
        step) in torch on the host cores, over a tenth of the parameters; the scaled
        gradients are restored before each call, outside the timing."""

        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        n = 120_000_000
        p = torch.nn.Parameter(self.p[:n].cpu())
        g_scaled = self.g_scaled[:n].cpu()
        p.grad = g_scaled.clone()
        opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
        scale = self.loss_scale

        def zero_step():
            g = p.grad
            found = torch.zeros((), dtype=torch.int32)
            if not torch.isfinite(g).all():
                found.fill_(1)
            if found.item():
                raise RuntimeError("unexpected overflow in the synthetic gradients")
            g.mul_(1.0 / scale)
            sq = torch.zeros((), dtype=torch.float32)
            sq.add_(g.detach().float().pow(2).sum())
            coef = 1.0 / (sq.sqrt() + 1e-6)
            if coef < 1:
                g.mul_(coef.to(dtype=g.dtype))
            opt.step()

        sec, calls = _time_cpu(zero_step, setup=lambda: p.grad.copy_(g_scaled))
        return dict(
            value=36 * n / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"{n:.1e} of 1.2e9 params (1/10): the ZeRO unscale_and_check_ + clip_grad_norm_(1.0) "
                   f"(zero.py:139-186) + torch.optim.AdamW(foreach=False).step() on CPU, scaled gradients "
                   f"restored untimed before each call, median of {calls} calls (~{CPU_TARGET_S:.0f} s) "
                   f"after 1 warm-up",
            seconds_per_call=sec, params_per_s=n / sec,
        )


class ModulesWorkload(Workload):
    """RMSNorm and SwiGLU forward + backward as picotron calls them: the ``RMSNorm`` module
    with ``use_triton_rmsnorm=True`` (reference src/picotron/models/picotron_decoder.py:32-46)
    and ``triton_swiglu`` inside ``SwiGLU.forward`` (src/picotron/nn/feedforward.py:26-43),
    each through autograd (``torch.autograd.grad`` to the inputs and the weight), against the
    same kernels called directly through the C ABI on preallocated buffers.  The value is the
    headline shapes' algorithmic bytes over the module path's wall time; ``config.paths``
    gives, per shape, the wall time per fwd+bwd call of both paths and the host time the
    module path spends issuing one call (measured without synchronising, so it shows where
    host work, not the kernels, sets the pace)."""

    name = "modules"
    metric = "RMSNorm/SwiGLU fwd+bwd through the module/autograd path, HBM GB/s & % of peak, 16k tok bf16"

    SHAPES = {
        # name: (rmsnorm shape, swiglu shape, dtype)
        "quickstart": ((2, 64, 128), (2, 64, 256), torch.float32),
        "headline": ((8, 2048, 4096), (8, 2048, 14336), torch.bfloat16),
    }

    def __init__(self, layers: int) -> None:
        from picotron_amd.nn.norm import RMSNorm

        self.layers = 1
        self.cases = {}
        for name, (rshape, sshape, dtype) in self.SHAPES.items():
            d = rshape[-1]
            norm = RMSNorm(d, eps=1e-5, use_triton_rmsnorm=True).to(device="cuda", dtype=dtype)
            norm_ref = RMSNorm(d, eps=1e-5).to(device="cuda", dtype=dtype)
            with torch.no_grad():
                norm.weight.copy_(_seeded((d,), dtype, 2, 0.02, 1.0))
                norm_ref.weight.copy_(norm.weight)
            case = dict(
                norm=norm,
                norm_ref=norm_ref,
                x=_seeded(rshape, dtype, 3).requires_grad_(True),
                dy=_seeded(rshape, dtype, 4),
                g=_seeded(sshape, dtype, 5).requires_grad_(True),
                u=_seeded(sshape, dtype, 6).requires_grad_(True),
                ds=_seeded(sshape, dtype, 7),
            )
            s = torch.finfo(dtype).bits // 8
            rows, cols = case["x"].numel() // d, d
            n = case["g"].numel()
            case["bytes"] = (2 * rows * cols * s + cols * s + 4 * rows) + (3 * rows * cols * s + 2 * cols * s + 4 * rows) \
                + 8 * n * s
            case["direct"] = self._direct(case, rows, cols, n, dtype)
            self.cases[name] = case
        self.bytes_per_step = self.cases["headline"]["bytes"]
        self.tokens_per_step = 16384
        self.dominant = "module path: rmsnorm fwd + bwd, swiglu fwd + bwd (5 kernels)"
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "RMSNorm(4096, use_triton_rmsnorm=True) on bf16 [8, 2048, 4096] (bf16 weight) and triton_swiglu on "
            "bf16 [8, 2048, 14336] gate/up, forward + torch.autograd.grad to inputs and weight; step = one call "
            "of each"
        )

    @staticmethod
    def _direct(case, rows, cols, n, dtype):
        """The same kernels through the C ABI on preallocated buffers (no autograd, no allocation)."""

        lib = _lib.lib()
        code = ops.dtype_code(dtype)
        x, dy, g, u, ds = (case[k].detach() for k in ("x", "dy", "g", "u", "ds"))
        w = case["norm"].weight.detach()
        y, dx, gy, dg, du = (torch.empty_like(t) for t in (x, x, g, g, g))
        rstd = torch.empty(rows, dtype=torch.float32, device="cuda")
        dw = torch.empty_like(w)
        ws_bytes = lib.pt_rmsnorm_bwd_workspace_bytes(rows, cols, code)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        keep = (y, dx, gy, dg, du, rstd, dw, ws)
        calls = [
            (lib.pt_rmsnorm_fwd, (_p(x), cols, _p(w), _p(y), cols, _p(rstd), rows, cols, ctypes.c_float(1e-5),
                                  code, code, stream)),
            (lib.pt_rmsnorm_bwd, (_p(dy), cols, _p(x), cols, _p(w), _p(rstd), _p(dx), cols, _p(dw), _p(ws),
                                  ws_bytes, rows, cols, code, code, stream)),
            (lib.pt_swiglu_fwd, (_p(g), _p(u), _p(gy), n, code, stream)),
            (lib.pt_swiglu_bwd, (_p(ds), _p(g), _p(u), _p(dg), _p(du), n, code, stream)),
        ]

        def run():
            for fn, args in calls:
                rc = fn(*args)
                if rc:
                    _lib.check(fn.__name__, rc)

        run.keep = keep
        return run

    @staticmethod
    def _module_call(case):
        from picotron_amd.nn.triton_kernels import triton_swiglu

        norm, x, g, u = case["norm"], case["x"], case["g"], case["u"]
        y = norm(x)
        torch.autograd.grad(y, (x, norm.weight), case["dy"])
        out = triton_swiglu(g, u)
        torch.autograd.grad(out, (g, u), case["ds"])

    @staticmethod
    def _fallback_call(case):
        """The same calls on the reference's PyTorch path (the modules with their flags off:
        the eager RMSNorm formula and ``F.silu(gate) * up``, autograd backwards)."""

        norm, x, g, u = case["norm_ref"], case["x"], case["g"], case["u"]
        y = norm(x)
        torch.autograd.grad(y, (x, norm.weight), case["dy"])
        out = F.silu(g) * u
        torch.autograd.grad(out, (g, u), case["ds"])

    def step(self, events):
        case = self.cases["headline"]
        if events is not None:
            start, end = events.pop()
            start.record()
        self._module_call(case)
        if events is not None:
            end.record()

    def extra(self, steps: int) -> dict:
        paths = {}
        for name, case in self.cases.items():
            reps = steps if name == "headline" else 50 * steps
            module = lambda: self._module_call(case)  # noqa: E731
            for _ in range(3):
                module()
                case["direct"]()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                module()
            t_issue = time.perf_counter() - t0
            torch.cuda.synchronize()
            t_module = time.perf_counter() - t0
            t0 = time.perf_counter()
            for _ in range(reps):
                case["direct"]()
            torch.cuda.synchronize()
            t_direct = time.perf_counter() - t0
            for _ in range(3):
                self._fallback_call(case)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                self._fallback_call(case)
            torch.cuda.synchronize()
            t_fallback = time.perf_counter() - t0
            paths[name] = {
                "rmsnorm_shape": list(case["x"].shape),
                "swiglu_shape": list(case["g"].shape),
                "dtype": str(case["x"].dtype).replace("torch.", ""),
                "calls": reps,
                "module_wall_us_per_call": round(t_module / reps * 1e6, 2),
                "module_host_issue_us_per_call": round(t_issue / reps * 1e6, 2),
                "direct_c_abi_wall_us_per_call": round(t_direct / reps * 1e6, 2),
                "reference_fallback_wall_us_per_call": round(t_fallback / reps * 1e6, 2),
                "module_gbs": round(case["bytes"] / (t_module / reps) / 1e9, 1),
                "direct_gbs": round(case["bytes"] / (t_direct / reps) / 1e9, 1),
            }
        return {"paths": paths}

    def cpu_baseline(self) -> dict:
        return None


class GradScalerStepWorkload(AdamWWorkload):
    """The train loop's single-GPU fp16 update (reference src/picotron/training/train_loop.py:
    155-160: GradScaler.unscale_, clip_grad_norm_, GradScaler.step, GradScaler.update), fused."""

    name = "fp16_step"
    metric = "Fused GradScaler unscale + inf-check + clip + AdamW step HBM GB/s & % of peak, 1.2e9 fp32 params"
    loss_scale = 1.0  # as in the ZeRO step workload: the gradients keep their magnitude

    def __init__(self, layers: int) -> None:
        super().__init__(layers)
        from picotron_amd.nn.triton_kernels import triton_grad_scaler_step

        n = self.n
        self.fn = triton_grad_scaler_step
        self.g.mul_(self.loss_scale)  # gradients as the scaled loss's backward leaves them
        self.g_scaled = self.g.clone()
        self.prm = torch.nn.Parameter(self.p)
        self.prm.grad = self.g
        self.opt = torch.optim.AdamW([self.prm], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
        self.scaler = torch.amp.GradScaler("cuda", init_scale=self.loss_scale)
        self.scaler.scale(torch.ones((), device="cuda"))  # the scale tensor, as scale(loss) makes it
        self.bytes_per_step = 36 * n  # stats: read g; step: read p, g, m, v, write p, m, v, g
        self.dominant = ("fused GradScaler step (grad_stats_kernel + grad_stats_finish_kernel, one host read "
                         "of the overflow flag, adamw_kernel with the combined unscale x clip multiplier, "
                         "the scaler's update)")
        self.dominant_bytes = self.bytes_per_step
        self.description = (
            "fp16 GradScaler update on one GPU: loss scale 1 (the written-back gradients keep their "
            "magnitude from step to step), finite check, unscale, "
            "clip_grad_norm_(1.0) (torch's rule) and the AdamW step, then the scaler's update; one flat "
            "1.2e9-element fp32 parameter; step = triton_grad_scaler_step (each step unscales and clips the "
            "gradients the previous one left)"
        )

    def step(self, events):
        if events is not None:
            start, end = events.pop()
            start.record()
        skipped = self.fn(self.scaler, self.opt, 1.0)
        if events is not None:
            end.record()
        if skipped:
            raise RuntimeError("unexpected overflow in the synthetic gradients")

    def extra(self, steps: int) -> dict:
        """torch's own sequence on the same data and its own AdamW (foreach, the default on a
        GPU): unscale_, clip_grad_norm_, step, update."""

        prm = torch.nn.Parameter(self.p.detach().clone())
        prm.grad = self.g_scaled.clone()
        opt = torch.optim.AdamW([prm], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
        scaler = torch.amp.GradScaler("cuda", init_scale=self.loss_scale)
        scaler.scale(torch.ones((), device="cuda"))

        def reference(_events=None):
            scaler.unscale_(opt)
            torch.nn.utils.clip_grad_norm_([prm], 1.0)
            scaler.step(opt)
            scaler.update()

        sec = _host_time(reference, steps)
        del prm, opt
        torch.cuda.empty_cache()
        return {"torch_sequence_ms_per_step": round(sec * 1e3, 4)}

    def cpu_baseline(self) -> dict:
        cores, _, _ = _cpu_info()
        torch.set_num_threads(cores)
        n = 120_000_000
        p = torch.nn.Parameter(self.p[:n].cpu())
        g_scaled = self.g_scaled[:n].cpu()
        p.grad = g_scaled.clone()
        opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
        scaler = torch.amp.GradScaler("cpu", init_scale=self.loss_scale)
        scaler.scale(torch.ones(()))

        def fp16_step():
            scaler.unscale_(opt)
            torch.nn.utils.clip_grad_norm_([p], 1.0)
            scaler.step(opt)
            scaler.update()

        sec, calls = _time_cpu(fp16_step, setup=lambda: p.grad.copy_(g_scaled))
        return dict(
            value=36 * n / sec / 1e9, unit="GB/s", cores=cores, kind="port",
            sample=f"{n:.1e} of 1.2e9 params (1/10): GradScaler.unscale_ + clip_grad_norm_(1.0) + "
                   f"GradScaler.step (torch.optim.AdamW(foreach=False)) + update on CPU, scaled gradients "
                   f"restored untimed before each call, median of {calls} calls (~{CPU_TARGET_S:.0f} s) "
                   f"after 1 warm-up",
            seconds_per_call=sec, params_per_s=n / sec,
        )


class CopyWorkload(Workload):
    name = "copy"
    metric = "128-bit streaming copy HBM GB/s (achievable-bandwidth reference)"
    dtype = "u8"
    nbytes = 1 << 30

    def __init__(self, layers: int) -> None:
        self.layers = layers
        self.launches_per_step = layers
        self.src = [torch.empty(self.nbytes, dtype=torch.uint8, device="cuda").fill_(i) for i in range(layers)]
        self.dst = [torch.empty(self.nbytes, dtype=torch.uint8, device="cuda") for _ in range(layers)]
        self.bytes_per_step = layers * 2 * self.nbytes
        self.tokens_per_step = 0
        self.dominant = "copy16_kernel"
        self.dominant_bytes = 2 * self.nbytes
        self.description = f"pt_copy of {layers} x 1 GiB buffers (read + write)"
        self.lib = _lib.lib()
        self.stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(self, events):
        for s, d in zip(self.src, self.dst):
            if events is not None:
                start, end = events.pop()
                start.record()
            rc = self.lib.pt_copy(_p(s), _p(d), self.nbytes, self.stream)
            if events is not None:
                end.record()
            if rc:
                _lib.check("pt_copy", rc)

    def cpu_baseline(self) -> dict:
        return None


# ------------------------------------------------------------------ whole training steps

# The reference's quickstart model and batch (src/picotron/config/picotron_decoder.yaml:7-10,
# 16-19): vocabulary 64, hidden 32, intermediate 64, 2 layers, 4 heads, sequence 16, micro-batch 2,
# learning rate 1e-3; AdamW betas (0.9, 0.999), eps 1e-8, weight decay 0 and no clipping are the
# config defaults (src/picotron/config/config.py:360-366,384-385); bf16 autocast is what
# `dtype: auto` resolves to on a bf16 GPU (train_loop.py:57,274-282).
QUICKSTART = dict(vocab=64, hidden=32, intermediate=64, layers=2, heads=4, kv_heads=4, seq=16, batch=2,
                  lr=1e-3, betas=(0.9, 0.999), weight_decay=0.0, clip=None, dtype="bf16",
                  theta=10_000.0, window=None, nope=(), tied=False)
# The notebook's pretraining run (examples/kaggle_demo_pretrain_sft_dpo.ipynb, cell 4): vocabulary
# 50257, hidden 20, intermediate 80, 8 layers, 2 heads over 1 key/value head, RoPE theta 1e6 except
# on layer 3, a 128-token sliding window, tied embeddings, sequence 256 x micro-batch 32, fp16
# with the train loop's GradScaler (train_loop.py:155-160), AdamW lr 3e-4, betas (0.9, 0.95),
# weight decay 0.1, gradients clipped to 1.0.
DEMO_1M = dict(vocab=50257, hidden=20, intermediate=80, layers=8, heads=2, kv_heads=1, seq=256, batch=32,
               lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, clip=1.0, dtype="fp16",
               theta=1e6, window=128, nope=(3,), tied=True)
QUICKSTART_VARIANTS = ("eager_reference", "eager_fused", "graph_reference", "graph_fused",
                       "graph_fused_residual")
# fp16 with a GradScaler: eager only (torch's GradScaler.step reads the overflow flag on the
# host every step; the captured fused fp16 step is switched off, see StepTrainer)
DEMO_VARIANTS = ("eager_reference", "eager_notebook_flags", "eager_fused")
STEP_VARIANTS = ("eager_reference", "eager_notebook_flags", "eager_fused", "graph_reference", "graph_fused",
                 "graph_fused_residual")
# the modules' kernel flags a variant turns on (``model.triton_kernels``); the notebook's config
# sets rmsnorm and swiglu and leaves rope, cross_entropy and adamw off
_MODULE_FLAGS = frozenset({"rmsnorm", "swiglu", "rope"})
_VARIANT_FLAGS = {"eager_reference": frozenset(), "graph_reference": frozenset(),
                  "eager_notebook_flags": frozenset({"rmsnorm", "swiglu"})}


class _StepBlock(torch.nn.Module):
    """The reference's decoder block (src/picotron/models/picotron_decoder.py:70-130): attention
    norm, causal self-attention (src/picotron/nn/attention.py: bias-free q/k/v/o projections,
    heads split to (B, H, S, D), RoPE on q and k unless the layer has none, key/value heads
    repeated for grouped-query attention, SDPA under a boolean causal or sliding-window mask),
    residual add, MLP norm, SwiGLU MLP, residual add.  The attention product runs in fp32 in
    every variant (plain PyTorch, identical between them)."""

    def __init__(self, cfg: dict, flags: frozenset, use_rope: bool) -> None:
        from picotron_amd.nn import RMSNorm, RotaryEmbedding, SwiGLU

        super().__init__()
        h, heads, kv = cfg["hidden"], cfg["heads"], cfg["kv_heads"]
        self.heads, self.kv_heads, self.head_dim, self.window = heads, kv, h // heads, cfg["window"]
        norm = "rmsnorm" in flags
        self.attention_norm = RMSNorm(h, use_triton_rmsnorm=norm)
        self.query_projection = torch.nn.Linear(h, h, bias=False)
        self.key_projection = torch.nn.Linear(h, kv * self.head_dim, bias=False)
        self.value_projection = torch.nn.Linear(h, kv * self.head_dim, bias=False)
        self.output_projection = torch.nn.Linear(h, h, bias=False)
        self.rotary_embedding = (RotaryEmbedding(self.head_dim, cfg["theta"], use_triton_rope="rope" in flags)
                                 if use_rope else None)
        self.mlp_norm = RMSNorm(h, use_triton_rmsnorm=norm)
        self.mlp = SwiGLU(h, cfg["intermediate"], use_triton_swiglu="swiglu" in flags)

    def _attention(self, x: torch.Tensor) -> torch.Tensor:
        b, s, h = x.shape
        split = lambda t, n: t.view(b, s, n, self.head_dim).transpose(1, 2)  # noqa: E731
        q = split(self.query_projection(x), self.heads)
        k = split(self.key_projection(x), self.kv_heads)
        v = split(self.value_projection(x), self.kv_heads)
        if self.rotary_embedding is not None:
            q, k = self.rotary_embedding(q, k)
        if self.kv_heads != self.heads:
            k = k.repeat_interleave(self.heads // self.kv_heads, dim=1)
            v = v.repeat_interleave(self.heads // self.kv_heads, dim=1)
        positions = torch.arange(s, device=x.device)
        mask = positions.unsqueeze(0) <= positions.unsqueeze(1)
        if self.window is not None:
            mask &= positions.unsqueeze(0) >= positions.unsqueeze(1) - self.window + 1
        out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask,
                                             scale=self.head_dim ** -0.5)
        return self.output_projection(out.to(q.dtype).transpose(1, 2).reshape(b, s, h))

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        hidden = hidden + self._attention(self.attention_norm(hidden))
        return hidden + self.mlp(self.mlp_norm(hidden))

    def forward_residual(self, hidden: torch.Tensor, normed: torch.Tensor, next_norm) -> tuple:
        """The same block with each residual add fused into the norm after it
        (``RMSNorm.add_and_norm``): takes the residual stream and this block's normed input,
        returns the stream and ``next_norm`` of it.  The autocast branch outputs are promoted
        to the stream's fp32 first, as the plain ``+`` promotes them."""

        attn = self._attention(normed).to(hidden.dtype)
        hidden, normed = self.mlp_norm.add_and_norm(attn, hidden)
        return next_norm.add_and_norm(self.mlp(normed).to(hidden.dtype), hidden)


class _StepDecoder(torch.nn.Module):
    """The reference's decoder (src/picotron/models/picotron_decoder.py:133-220) with RoPE
    positions, built from this package's modules; ``flags`` names the modules whose kernel flag
    is on ("rmsnorm", "swiglu", "rope"), as ``model.triton_kernels`` sets them.  A tied output
    projection uses the token embeddings' weight (`TiedOutputProjection`,
    picotron_decoder.py:49-67)."""

    def __init__(self, cfg: dict, flags: frozenset, residual: bool = False) -> None:
        from picotron_amd.nn import RMSNorm

        super().__init__()
        self.residual = residual
        v, h = cfg["vocab"], cfg["hidden"]
        self.token_embeddings = torch.nn.Embedding(v, h)
        self.layers = torch.nn.ModuleList(_StepBlock(cfg, flags, i not in cfg["nope"])
                                          for i in range(cfg["layers"]))
        self.final_norm = RMSNorm(h, use_triton_rmsnorm="rmsnorm" in flags)
        self.output_projection = None if cfg["tied"] else torch.nn.Linear(h, v, bias=False)

    def _project(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.output_projection is None:
            return F.linear(hidden, self.token_embeddings.weight)
        return self.output_projection(hidden)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        hidden = self.token_embeddings(input_ids)
        if self.residual:
            normed = self.layers[0].attention_norm(hidden)
            norms = [layer.attention_norm for layer in self.layers[1:]] + [self.final_norm]
            for layer, next_norm in zip(self.layers, norms):
                hidden, normed = layer.forward_residual(hidden, normed, next_norm)
            return self._project(normed)
        for layer in self.layers:
            hidden = layer(hidden)
        return self._project(self.final_norm(hidden))


class StepTrainer:
    """One training step of a decoder config as the train loop runs it
    (src/picotron/training/train_loop.py:134-168): zero_grad, forward and the next-token loss on
    the (B, V, S-1) logits view under autocast, backward, then the update: the plain branch
    (clip if configured, optimizer step; :165-168) or, for fp16, the GradScaler branch (scale,
    backward, unscale_, clip, step, update; :155-160).

    ``variant``: ``eager_reference`` runs the modules with their kernel flags off, torch's loss
    and torch's update (the reference's fallbacks); ``eager_notebook_flags`` turns on the flags
    the notebook demo sets (RMSNorm and SwiGLU); ``eager_fused`` every flag (also RoPE), with
    ``CrossEntropyWithFallback(use_triton=True)`` and the fused update of
    ``AdamWStepWithFallback`` (``step(optimizer, max_grad_norm=)`` or ``step_with_grad_scaler``);
    the ``graph_*`` variants (bf16 configs) capture the whole step in one HIP graph
    (capturable AdamW, gradients zeroed in place so that their addresses stay fixed) and
    replay it; ``graph_fused_residual`` also fuses each residual add into the norm after it
    (``RMSNorm.add_and_norm``), a change to the model's code rather than a flag.
    ``capturable`` overrides the optimizer's flag (by default set for the graph variants)."""

    def __init__(self, cfg: dict, variant: str, seed: int = 1337, capturable: bool | None = None) -> None:
        from picotron_amd.nn.triton_kernels import AdamWStepWithFallback, CrossEntropyWithFallback

        if variant not in STEP_VARIANTS:
            raise ValueError(f"unknown variant {variant}")
        self.cfg, self.variant = cfg, variant
        self.graphed = variant.startswith("graph")
        flags = _VARIANT_FLAGS.get(variant, _MODULE_FLAGS)
        self.fused_update = "fused" in variant
        if self.graphed and cfg["dtype"] == "fp16":
            # torch's GradScaler.step reads its overflow flag on the host; the fused update
            # decides on the device and captures (a whole captured update is tested), but the
            # captured fp16 decoder step is switched off: its first run took a host
            # segmentation fault in the autograd worker thread, whose cause is not found
            raise ValueError("a captured fp16 step is switched off (see the comment above)")
        self.autocast = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float16
        torch.manual_seed(seed)
        self.model = _StepDecoder(cfg, flags, residual=variant.endswith("residual")).cuda()
        self.optimizer = torch.optim.AdamW(self.model.parameters(), lr=cfg["lr"], betas=cfg["betas"],
                                           eps=1e-8, weight_decay=cfg["weight_decay"],
                                           capturable=self.graphed if capturable is None else capturable)
        self.scaler = torch.amp.GradScaler("cuda") if cfg["dtype"] == "fp16" else None
        self.loss_function = CrossEntropyWithFallback(use_triton=self.fused_update)
        self.optimizer_step = AdamWStepWithFallback(use_triton=self.fused_update)
        self.graph = None
        self.static_ids = None

    def _step(self, input_ids: torch.Tensor) -> torch.Tensor:
        clip = self.cfg["clip"]
        self.optimizer.zero_grad(set_to_none=not self.graphed)
        with torch.autocast("cuda", dtype=self.autocast, cache_enabled=not self.graphed):
            logits = self.model(input_ids)
            loss = self.loss_function(logits[:, :-1, :].transpose(1, 2), input_ids[:, 1:])
        if self.scaler is not None:
            self.scaler.scale(loss).backward()
            if self.fused_update:
                self.optimizer_step.step_with_grad_scaler(self.scaler, self.optimizer, clip)
            else:
                self.scaler.unscale_(self.optimizer)
                if clip is not None:
                    torch.nn.utils.clip_grad_norm_(self.model.parameters(), clip)
                self.scaler.step(self.optimizer)
                self.scaler.update()
        else:
            loss.backward()
            if self.fused_update and clip is not None:
                self.optimizer_step.step(self.optimizer, max_grad_norm=clip)
            else:
                if clip is not None:
                    torch.nn.utils.clip_grad_norm_(self.model.parameters(), clip)
                self.optimizer_step.step(self.optimizer)
        return loss.detach()

    def prepare(self, input_ids: torch.Tensor, warmup: int = 3) -> None:
        """Warm-up steps (optimizer state, cached tables), then the capture for a graph
        variant.  Fails if a fused module fell back to PyTorch."""

        import warnings

        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            if self.graphed:
                self.static_ids = input_ids.clone()
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    for _ in range(warmup):
                        self._step(self.static_ids)
                torch.cuda.current_stream().wait_stream(side)
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self.static_loss = self._step(self.static_ids)
            else:
                for _ in range(warmup):
                    self._step(input_ids)
            torch.cuda.synchronize()
        fallbacks = [str(w.message) for w in caught if "unavailable" in str(w.message)]
        if fallbacks:
            raise RuntimeError(f"{self.variant}: a fused kernel fell back to PyTorch: {fallbacks[0]}")

    def step(self, input_ids: torch.Tensor) -> torch.Tensor:
        if self.graph is None:
            return self._step(input_ids)
        self.static_ids.copy_(input_ids)
        self.graph.replay()
        return self.static_loss


class QuickstartTrainer(StepTrainer):
    """:class:`StepTrainer` on the quickstart config."""

    def __init__(self, variant: str, seed: int = 1337, capturable: bool | None = None) -> None:
        super().__init__(QUICKSTART, variant, seed, capturable)


def _describe(cfg: dict) -> str:
    return (f"vocab {cfg['vocab']}, hidden {cfg['hidden']}, intermediate {cfg['intermediate']}, "
            f"{cfg['layers']} layers, {cfg['heads']} heads / {cfg['kv_heads']} key-value heads, "
            f"micro-batch {cfg['batch']} x sequence {cfg['seq']}, {cfg['dtype']} autocast"
            + (", GradScaler" if cfg["dtype"] == "fp16" else "")
            + (f", clip {cfg['clip']}" if cfg["clip"] is not None else "")
            + (f", sliding window {cfg['window']}" if cfg["window"] else "")
            + (", tied embeddings" if cfg["tied"] else ""))


def _quickstart_line(steps: int) -> dict:
    """The quickstart step figures with what they describe (a section of the default line)."""

    return {
        "workload": ("one training step of the quickstart decoder (" + _describe(QUICKSTART) + "): zero_grad, "
                     "forward, next-token loss on the (B, V, S-1) view, backward, AdamW step; batches resident "
                     "on the device"),
        "steps": steps,
        "variants": step_figures(QUICKSTART, steps, QUICKSTART_VARIANTS),
    }


def _demo_line(steps: int) -> dict:
    """The notebook demo's step figures with what they describe (a section of the default line)."""

    return {
        "workload": ("one training step of the notebook's pretraining model (" + _describe(DEMO_1M) + "): "
                     "zero_grad, forward, next-token loss on the (B, V, S-1) view, scaled backward, unscale + "
                     "clip + AdamW step + scaler update; batches resident on the device"),
        "steps": steps,
        "variants": step_figures(DEMO_1M, steps, DEMO_VARIANTS),
    }


def step_figures(cfg: dict, steps: int, variants) -> dict:
    """Per variant: the host time to issue one step, the wall time per step when steps are
    issued back to back (the slower of host and device sets it), the device time per step
    between HIP events around those steps, and the wall time per step in the train loop's own
    form, which reads the loss back after every step (train_loop.py:169)."""

    g = torch.Generator(device="cuda").manual_seed(5)
    batches = torch.randint(0, cfg["vocab"], (steps, cfg["batch"], cfg["seq"]), generator=g, device="cuda")
    out = {}
    for variant in variants:
        trainer = StepTrainer(cfg, variant)
        trainer.prepare(batches[0])
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for i in range(steps):
            trainer.step(batches[i])
        end.record()
        issued = time.perf_counter() - t0
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        t0 = time.perf_counter()
        for i in range(steps):
            trainer.step(batches[i]).item()
        loop = time.perf_counter() - t0
        out[variant] = {
            "host_issue_us_per_step": round(issued / steps * 1e6, 1),
            "wall_us_per_step": round(wall / steps * 1e6, 1),
            "device_us_per_step": round(start.elapsed_time(end) / steps * 1e3, 1),
            "train_loop_us_per_step": round(loop / steps * 1e6, 1),
        }
        del trainer
        torch.cuda.empty_cache()
    return out


WORKLOADS = {
    "headline": HeadlineWorkload,
    "rmsnorm": RMSNormWorkload,
    "rmsnorm_fp32": RMSNormFp32Workload,
    "residual_rmsnorm": ResidualRMSNormWorkload,
    "swiglu": SwiGLUWorkload,
    "rope": RoPEWorkload,
    "ce": CrossEntropyWorkload,
    "ce_train": CrossEntropyTrainWorkload,
    "ce_ref_call": CrossEntropyReferenceCallWorkload,
    "ce_train_fp16": CrossEntropyTrainFp16Workload,
    "ce_demo_fp16": CrossEntropyDemoFp16Workload,
    "adamw": AdamWWorkload,
    "adamw_list": AdamWListWorkload,
    "adamw_clip": AdamWClipWorkload,
    "zero_step": ZeroMixedPrecisionStepWorkload,
    "fp16_step": GradScalerStepWorkload,
    "modules": ModulesWorkload,
    "copy": CopyWorkload,
}

DEFAULT_LAYERS = {"headline": 4, "rmsnorm": 4, "rmsnorm_fp32": 4, "ce_ref_call": 1, "residual_rmsnorm": 4, "swiglu": 2, "rope": 4, "ce": 1, "ce_train": 1, "ce_train_fp16": 1, "ce_demo_fp16": 1, "adamw": 1, "adamw_list": 1, "adamw_clip": 1,
                  "zero_step": 1, "fp16_step": 1, "modules": 1, "copy": 4}


def _traffic(workload: str) -> dict | None:
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter
    summary (profiles/<workload>_traffic.json), if one exists."""

    path = ROOT / "profiles" / f"{workload}_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    return data


def _measure(wl: Workload, name: str, steps: int, warmup: int) -> dict:
    """Times ``steps`` steps of ``wl`` after ``warmup`` untimed ones.

    Pass 1 (the value): nothing but the workload's own launches between two device
    synchronisations, host clock.  Pass 2 (the roofline): the same steps again with a HIP
    event pair around every timed launch, recorded on the stream the kernels run on; the
    event records add a few microseconds per launch, so this pass is not used for the value.
    A workload with several launch kinds (timed_kinds) gets one event list per kind; the
    others time their dominant launch.  Per-launch HBM traffic comes from the committed
    counter summary (profiles/<name>_traffic.json) when there is one."""

    for _ in range(warmup):
        wl.step(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.step(None)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    kinds = getattr(wl, "timed_kinds", None)
    if kinds is None:
        kinds = {"dominant": wl.launches_per_step}
    events = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(steps * n)] for k, n in kinds.items()}
    pending = {k: list(reversed(v)) for k, v in events.items()}
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        wl.step(pending if hasattr(wl, "timed_kinds") else pending["dominant"])
    torch.cuda.synchronize()
    elapsed_instrumented = time.perf_counter() - t1

    traffic = _traffic(name)
    per_kernel = {}
    for kind, pairs in events.items():
        launch_ms = [a.elapsed_time(b) for a, b in pairs]
        info = wl.kinds[kind] if kind in getattr(wl, "kinds", {}) else {"kernel": wl.dominant,
                                                                         "bytes": wl.dominant_bytes}
        avg_us = statistics.mean(launch_ms) * 1e3
        achieved = info["bytes"] / (avg_us * 1e-6) / 1e9
        entry = {
            "kernel": info["kernel"],
            "algorithmic_bytes_per_launch": info["bytes"],
            "avg_launch_us": round(avg_us, 2),
            "median_launch_us": round(statistics.median(launch_ms) * 1e3, 2),
            "launches_timed": len(launch_ms),
            "achieved": round(achieved, 1),
            "frac": round(achieved / PEAK_GBPS, 4),
            "traffic": None,
            "total_ms": sum(launch_ms),
        }
        if traffic:
            per = traffic.get("kernels", {}).get(kind) if "kernels" in traffic and isinstance(traffic["kernels"], dict) else traffic
            if per:
                entry["traffic"] = per.get("bytes_per_launch")
        per_kernel[kind] = entry
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["total_ms"])
    return dict(elapsed=elapsed, elapsed_instrumented=elapsed_instrumented, per_kernel=per_kernel,
                dominant=dominant, traffic_source=traffic.get("source") if traffic else None,
                steps=steps)


def _roofline(m: dict) -> dict:
    dom = m["per_kernel"][m["dominant"]]
    roofline = {
        "bound": "hbm",
        "achieved": dom["achieved"],
        "peak": PEAK_GBPS,
        "unit": "GB/s",
        "frac": dom["frac"],
        "traffic": dom["traffic"],
        "kernel": dom["kernel"],
        "algorithmic_bytes_per_launch": dom["algorithmic_bytes_per_launch"],
        "avg_launch_us": dom["avg_launch_us"],
        "median_launch_us": dom["median_launch_us"],
        "launches_timed": dom["launches_timed"],
        "timing": "HIP events around each launch, in a second pass of the same steps",
        "ms_per_step_with_events": round(m["elapsed_instrumented"] / m["steps"] * 1e3, 4),
    }
    if m["traffic_source"]:
        roofline["traffic_source"] = m["traffic_source"]
    if len(m["per_kernel"]) > 1:
        roofline["per_kernel"] = {k: {kk: vv for kk, vv in v.items() if kk != "total_ms"}
                                  for k, v in m["per_kernel"].items()}
    return roofline


def _cpu_line(wl: Workload) -> dict | None:
    cpu = wl.cpu_baseline()
    if cpu is not None:
        cores, ncpu, model = _cpu_info()
        cpu.update(os_cpu_count=ncpu, cpu_model=model)
        for key in ("value", "seconds_per_call", "tokens_per_s", "params_per_s"):
            if key in cpu:
                cpu[key] = round(cpu[key], 4) if key == "seconds_per_call" else round(cpu[key], 2)
    return cpu


# ------------------------------------------------------------------ cross-entropy by vocabulary

# Vocabularies that start rows on 128-byte lines (multiples of 64 16-bit logits) and ones that
# do not: odd (GPT-2's 50257), multiples of 8 and 16 (rows on 16-byte boundaries), and the
# common model vocabularies around them.
CE_VOCABS = (32000, 32001, 32008, 48000, 50256, 50257, 50304, 57000, 64000, 128256, 128264, 151936)


def ce_vocab_figures(rows: int = 8160, vocabs=CE_VOCABS, steps: int = 20) -> dict:
    """Per vocabulary, [rows, V] logits: the bf16 forward writing the gradient in place and
    the fp16 forward (log-sum-exps only) and backward (the gradient at a GradScaler-sized
    scale, in place), each timed with HIP events over ``steps`` calls after 3 warm-up calls;
    GB/s on the algorithmic bytes (bf16: read + write; fp16: read, then read + write)."""

    from picotron_amd import ops

    g = torch.Generator(device="cuda").manual_seed(0)

    def timed(fn) -> float:
        for _ in range(3):
            fn()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps * 1e3

    out = {}
    for v in vocabs:
        targets = torch.randint(0, v, (rows,), device="cuda", generator=g)
        row = {"line_aligned": (v * 2) % 128 == 0}
        buf = (torch.randn(rows, v, device="cuda", generator=g) * 2).to(torch.bfloat16)
        us = timed(lambda: ops.cross_entropy(buf, targets, write_grad=True))
        row["bf16_forward_us"] = round(us, 1)
        row["bf16_forward_gbs"] = round(2 * rows * v * 2 / us / 1e3, 1)
        del buf
        buf = (torch.randn(rows, v, device="cuda", generator=g) * 2).to(torch.float16)
        state = {}

        def forward():
            state["ws"] = ops.cross_entropy(buf, targets, write_grad=True)[1]

        us = timed(forward)
        row["fp16_forward_us"] = round(us, 1)
        row["fp16_forward_gbs"] = round(rows * v * 2 / us / 1e3, 1)
        scale = torch.full((), 65536.0, device="cuda")
        us = timed(lambda: ops.cross_entropy_scale_grad(buf, targets, scale, workspace=state["ws"]))
        row["fp16_backward_us"] = round(us, 1)
        row["fp16_backward_gbs"] = round(2 * rows * v * 2 / us / 1e3, 1)
        del buf, state
        torch.cuda.empty_cache()
        out[str(v)] = row
    return out


def _ce_vocabs_main(args) -> int:
    """The cross-entropy kernels across vocabularies as one line: value = the lowest bf16
    forward GB/s of the list (the figure row alignment moves most)."""

    rows = 8160
    figs = ce_vocab_figures(rows, CE_VOCABS, args.steps)
    worst = min(f["bf16_forward_gbs"] for f in figs.values())
    result = {
        "metric": "cross-entropy GB/s by vocabulary, [8160, V] (lowest bf16 forward of the list)",
        "value": worst,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": 3,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16/f16",
        "data": "synthetic (seeded on device)",
        "config": {"workload": f"{rows} rows x V logits, in place; HIP events per call", "parallelism": "single GPU",
                   "vocabularies": figs},
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(result))
    return 0


def _step_main(args) -> int:
    """A whole training step as its own line: value = tokens per second of the lead variant
    (the graph-captured fused step for the quickstart model, the fused eager step for the
    notebook's fp16 model) or of the one variant asked for, steps issued back to back."""

    demo = args.workload == "demo_step"
    cfg, allowed = (DEMO_1M, DEMO_VARIANTS) if demo else (QUICKSTART, QUICKSTART_VARIANTS)
    if args.variant != "all" and args.variant not in allowed:
        print(f"{args.workload}: variant {args.variant} is not one of {', '.join(allowed)}", file=sys.stderr)
        return 2
    variants = allowed if args.variant == "all" else (args.variant,)
    describe = _demo_line if demo else _quickstart_line
    line = describe(args.steps) if args.variant == "all" else {
        "steps": args.steps, "variants": step_figures(cfg, args.steps, variants)}
    figs = line["variants"]
    lead = next((v for v in ("graph_fused", "eager_fused") if v in figs), variants[0])
    us = figs[lead]["wall_us_per_step"]
    tokens = cfg["batch"] * cfg["seq"]
    name = "notebook demo decoder" if demo else "quickstart decoder"
    result = {
        "metric": f"{name} training step ({lead}), tokens/s",
        "value": round(tokens / (us * 1e-6), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": 3,
        "ms_per_step": round(us * 1e-3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic token ids (seeded on device)",
        "config": {"tokens_per_step": tokens, "parallelism": "single GPU", **line},
        # a few microseconds of work per kernel: launch latency, not HBM, bounds these steps
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(result))
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description="fused-kernel HBM benchmark (one MI355X)")
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=sorted([*WORKLOADS, "quickstart_step", "demo_step", "ce_vocabs"]),
                        default="headline")
    parser.add_argument("--variant", choices=("all", *STEP_VARIANTS), default="all",
                        help="quickstart_step and demo_step only: the step variant(s) to time")
    parser.add_argument("--layers", type=int, default=None)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extra", action="store_true",
                        help="skip the workload's comparison measurements (e.g. the unfused "
                             "sequence and the other configurations), so that a profile holds "
                             "only the timed launches")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the kernels run on a single MI355X and the library has "
              "no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if "PICOTRON_HIP_LIB" not in os.environ:
        from picotron_amd.build import ensure_built

        ensure_built()  # only when the in-tree library is missing
    _lib.lib()
    if not ops.device_supported(0):
        print("GPU 0 is not a gfx950 (MI355X) device", file=sys.stderr)
        return 2

    if args.workload in ("quickstart_step", "demo_step"):
        return _step_main(args)
    if args.workload == "ce_vocabs":
        return _ce_vocabs_main(args)
    global _WITH_CPU_BASELINE
    _WITH_CPU_BASELINE = not args.no_cpu_baseline
    layers = args.layers or DEFAULT_LAYERS[args.workload]
    wl = WORKLOADS[args.workload](layers)
    torch.cuda.synchronize()

    m = _measure(wl, args.workload, args.steps, args.warmup)
    elapsed = m["elapsed"]
    ms_per_step = elapsed / args.steps * 1e3
    gbps = wl.bytes_per_step / (elapsed / args.steps) / 1e9
    roofline = _roofline(m)

    extra = None if args.no_extra else wl.extra(args.steps)
    cpu = None if args.no_cpu_baseline else _cpu_line(wl)

    result = {
        "metric": wl.metric,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic (seeded on device)",
        "config": {
            "workload": wl.description,
            "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
            "algorithmic_bytes_per_step": wl.bytes_per_step,
            "tokens_per_step": wl.tokens_per_step,
            "tokens_per_s": round(wl.tokens_per_step / (elapsed / args.steps), 1),
            "layers_per_step": layers,
            "parallelism": "single GPU",
            **(extra or {}),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
