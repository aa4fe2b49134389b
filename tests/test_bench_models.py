"""The whole-step models bench.py times, checked on the CPU with the kernel flags off (the
modules' PyTorch paths): the notebook demo's decoder keeps the reference's attention
semantics (src/picotron/nn/attention.py: causal, a sliding window of 128 keys, key/value
heads shared by grouped queries; src/picotron/models/picotron_decoder.py: no RoPE on the
`nope` layers, an output projection tied to the token embeddings), checked as properties of
the outputs; and the command line refuses what it does not measure."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

import bench

ROOT = Path(__file__).resolve().parent.parent
NONE = frozenset()


def _demo(seq=160, layers=2, nope=(1,), window=None):
    cfg = dict(bench.DEMO_1M, seq=seq, layers=layers, nope=nope, vocab=97)
    cfg["window"] = cfg["window"] if window is None else window
    torch.manual_seed(0)
    return cfg, bench._StepDecoder(cfg, NONE).double()


def test_demo_decoder_shapes_and_modules():
    cfg, model = _demo()
    assert model.output_projection is None  # tied to the token embeddings
    assert model.layers[0].rotary_embedding is not None and model.layers[1].rotary_embedding is None
    block = model.layers[0]
    assert block.key_projection.out_features == cfg["kv_heads"] * block.head_dim  # one key/value head
    ids = torch.randint(0, cfg["vocab"], (2, cfg["seq"]))
    assert model(ids).shape == (2, cfg["seq"], cfg["vocab"])


def test_demo_attention_is_causal_and_windowed():
    """Changing token j changes no output before j (causal), and with one layer no output at
    or past j + window (the sliding window of 128 keys); it does change the outputs in between."""

    cfg, model = _demo(seq=200, layers=1, nope=())
    ids = torch.randint(0, cfg["vocab"], (1, cfg["seq"]))
    j = 20
    other = ids.clone()
    other[0, j] = (ids[0, j] + 1) % cfg["vocab"]
    with torch.no_grad():
        a, b = model(ids), model(other)
    diff = (a - b).abs().amax(dim=-1)[0]
    window = cfg["window"]
    assert float(diff[:j].max()) == 0.0
    assert float(diff[j:j + window].min()) > 0.0
    assert float(diff[j + window:].max()) == 0.0


def test_tied_projection_gradient_collects_both_uses():
    cfg, model = _demo(seq=16)
    ids = torch.randint(0, cfg["vocab"], (2, cfg["seq"]))
    logits = model(ids)
    torch.nn.functional.cross_entropy(logits[:, :-1, :].transpose(1, 2), ids[:, 1:]).backward()
    grad = model.token_embeddings.weight.grad
    # rows of tokens that never occur get a gradient only from the output projection
    unused = sorted(set(range(cfg["vocab"])) - set(ids.flatten().tolist()))
    assert unused and float(grad[unused].abs().max()) > 0.0


def test_fp16_capture_is_switched_off_and_unknown_variants_rejected():
    with pytest.raises(ValueError, match="switched off"):
        bench.StepTrainer(bench.DEMO_1M, "graph_fused")
    with pytest.raises(ValueError, match="unknown variant"):
        bench.StepTrainer(bench.QUICKSTART, "graph_everything")
    assert set(bench.DEMO_VARIANTS) <= set(bench.STEP_VARIANTS)
    assert not any(v.startswith("graph") for v in bench.DEMO_VARIANTS)


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 2 and "one GPU" in out.stderr
