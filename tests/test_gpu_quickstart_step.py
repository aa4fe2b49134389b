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



def test_residual_fused_model_takes_the_same_steps(gpu):
    """The model with each residual add fused into the norm after it computes the same steps
    as the plain model (the adds are the same fp32 adds; the norms may round differently)."""

    batches = _batches(6)
    plain, fused = QuickstartTrainer("graph_fused"), QuickstartTrainer("graph_fused_residual")
    plain.prepare(batches[0])
    fused.prepare(batches[0])
    for i in range(1, 6):
        loss_p = plain.step(batches[i]).clone()
        loss_f = fused.step(batches[i])
        torch.cuda.synchronize()
        torch.testing.assert_close(loss_f, loss_p, rtol=1e-4, atol=1e-5, msg=f"step {i}")
    for (name, a), b in zip(fused.model.named_parameters(), plain.model.parameters()):
        torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-4, atol=1e-5, msg=name)
