"""The quickstart training step that bench.py times (the reference's quickstart decoder,
src/picotron/config/picotron_decoder.yaml:7-10, one train-loop step under bf16 autocast):
replaying its HIP graph computes what the same steps compute eagerly, for the fused modules
and for the reference's fallbacks."""

from __future__ import annotations

import pytest
import torch

from bench import QUICKSTART, QuickstartTrainer

pytestmark = pytest.mark.gpu


def _batches(n: int) -> torch.Tensor:
    g = torch.Generator(device="cuda").manual_seed(11)
    return torch.randint(0, QUICKSTART["vocab"], (n, QUICKSTART["batch"], QUICKSTART["seq"]),
                         generator=g, device="cuda")


@pytest.mark.parametrize("kind", ["fused", "reference"])
def test_graph_replays_match_eager_steps(gpu, kind):
    batches = _batches(6)
    graphed = QuickstartTrainer(f"graph_{kind}")
    eager = QuickstartTrainer(f"eager_{kind}", capturable=True)
    graphed.prepare(batches[0])
    eager.prepare(batches[0])
    for i in range(1, 6):
        loss_g = graphed.step(batches[i]).clone()
        loss_e = eager.step(batches[i])
        torch.cuda.synchronize()
        torch.testing.assert_close(loss_g, loss_e, rtol=1e-5, atol=1e-6, msg=f"step {i}")
    for (name, a), b in zip(graphed.model.named_parameters(), eager.model.parameters()):
        torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-5, atol=1e-6, msg=name)

