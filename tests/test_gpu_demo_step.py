"""The notebook demo's training step that bench.py times (examples/kaggle_demo_pretrain_sft_dpo.ipynb,
cell 4: tied embeddings, grouped-query attention, a sliding window, one layer without RoPE, fp16
with the train loop's GradScaler, clipping at 1.0): the step with the notebook's own flags
(RMSNorm and SwiGLU), and with every flag on (also RoPE, the fused cross-entropy and the fused
scaler + clip + AdamW update), follows the reference's fallbacks step for step."""

from __future__ import annotations

import pytest
import torch

from bench import DEMO_1M, StepTrainer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant", ["eager_notebook_flags", "eager_fused"])
def test_demo_steps_follow_the_reference(gpu, variant):
    g = torch.Generator(device="cuda").manual_seed(23)
    batches = torch.randint(0, DEMO_1M["vocab"], (6, DEMO_1M["batch"], DEMO_1M["seq"]),
                            generator=g, device="cuda")
    reference, other = StepTrainer(DEMO_1M, "eager_reference"), StepTrainer(DEMO_1M, variant)
    initial = [p.detach().clone() for p in reference.model.parameters()]
    reference.prepare(batches[0])
    other.prepare(batches[0])
    for i in range(1, 6):
        loss_r = float(reference.step(batches[i]))
        loss_o = float(other.step(batches[i]))
        print(f"{variant} step {i}: loss {loss_o:.6f} against {loss_r:.6f}", flush=True)
        # fp16 kernels round differently from torch's: the losses agree to fp16's resolution
        assert abs(loss_o - loss_r) <= 2e-3 * abs(loss_r), f"step {i}: {loss_o} against {loss_r}"
    assert other.scaler.get_scale() == reference.scaler.get_scale()
    # parameters: the two runs' difference is small against how far the steps moved them
    # (elementwise, an Adam update of a near-zero gradient may flip sign under rounding)
    for (name, p_o), p_r, p0 in zip(other.model.named_parameters(), reference.model.parameters(), initial):
        moved = float((p_r.detach() - p0).abs().mean())
        apart = float((p_o.detach() - p_r.detach()).abs().mean())
        assert moved > 0, name
        assert apart <= 0.05 * moved, f"{name}: mean |difference| {apart} against mean |update| {moved}"


@pytest.mark.skip(reason="switched off: the first run took a host segmentation fault in the autograd "
                         "worker thread (the eager step's backward right after the first replay; no GPU "
                         "fault); its cause is not found, so the captured fp16 decoder step stays off. The "
                         "captured fp16 update itself is tested in test_gpu_grad_scaler.py")
def test_graph_replays_match_eager_steps(gpu):
    """The fused fp16 step captured in one HIP graph (its GradScaler update decides each
    step's overflow on the device) computes what the same steps compute eagerly with a
    capturable optimizer."""

    g = torch.Generator(device="cuda").manual_seed(29)
    batches = torch.randint(0, DEMO_1M["vocab"], (6, DEMO_1M["batch"], DEMO_1M["seq"]),
                            generator=g, device="cuda")
    graphed = StepTrainer(DEMO_1M, "graph_fused")
    eager = StepTrainer(DEMO_1M, "eager_fused", capturable=True)
    graphed.prepare(batches[0])
    eager.prepare(batches[0])
    for i in range(1, 6):
        loss_g = graphed.step(batches[i]).clone()
        loss_e = eager.step(batches[i])
        torch.cuda.synchronize()
        print(f"captured demo step {i}: loss {float(loss_g):.6f} against {float(loss_e):.6f}", flush=True)
        torch.testing.assert_close(loss_g, loss_e, rtol=1e-5, atol=1e-6, msg=f"step {i}")
    assert graphed.scaler.get_scale() == eager.scaler.get_scale()
    for (name, a), b in zip(graphed.model.named_parameters(), eager.model.parameters()):
        torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-5, atol=1e-6, msg=name)
