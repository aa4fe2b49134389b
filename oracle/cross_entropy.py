"""Cross-entropy oracle (test infrastructure; see oracle/__init__.py).

Reference: src/picotron/nn/triton_kernels/cross_entropy.py:97-109 falls back to
F.cross_entropy(logits, targets): mean over targets != -100 of lse(row) - row[target];
its gradient is (softmax - onehot(target)) / n_valid on kept rows and 0 on ignored rows.
Rows may come as (N, C) or (N, C, d) (class dim 1), as F.cross_entropy accepts.
"""

from __future__ import annotations

import torch
from torch import Tensor


def _rows(logits: Tensor, targets: Tensor) -> tuple[Tensor, Tensor]:
    if logits.dim() == 3:
        return logits.transpose(1, 2).reshape(-1, logits.size(1)), targets.reshape(-1)
    return logits, targets


def forward_backward(
    logits: Tensor, targets: Tensor, ignore_index: int = -100, compute: torch.dtype = torch.float64
) -> tuple[Tensor, Tensor]:
    """(loss, dlogits) in ``compute``; dlogits has the logits' shape."""

    rows, tgt = _rows(logits.to(compute), targets)
    keep = tgt != ignore_index
    n_valid = keep.sum().to(compute)
    mx = rows.max(dim=-1, keepdim=True).values
    lse = mx.squeeze(-1) + torch.log(torch.exp(rows - mx).sum(dim=-1))
    safe_t = torch.where(keep, tgt, torch.zeros_like(tgt))
    picked = rows.gather(1, safe_t.unsqueeze(1)).squeeze(1)
    per_row = torch.where(keep, lse - picked, torch.zeros_like(lse))
    loss = per_row.sum() / n_valid
    grad = torch.exp(rows - lse.unsqueeze(-1))
    grad.scatter_add_(1, safe_t.unsqueeze(1), -torch.ones_like(picked).unsqueeze(1))
    grad = torch.where(keep.unsqueeze(1), grad / n_valid, torch.zeros_like(grad))
    if logits.dim() == 3:
        b, c, d = logits.shape
        grad = grad.reshape(b, d, c).transpose(1, 2)
    return loss, grad


def fallback_forward_backward(logits: Tensor, targets: Tensor) -> tuple[Tensor, Tensor]:
    """The reference's fallback as the train loop runs it under autocast: F.cross_entropy on
    fp32-upcast logits, forward and autograd backward.  Returns (loss fp32, dlogits fp32)."""

    lf = logits.detach().float().requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(lf, targets)
    loss.backward()
    return loss.detach(), lf.grad


def shifted_forward_backward(
    logits: Tensor, input_ids: Tensor, ignore_index: int = -100, compute: torch.dtype = torch.float64
) -> tuple[Tensor, Tensor]:
    """The train loop's next-token loss on (B, S, V) logits (reference
    src/picotron/training/train_loop.py:141-144: ``logits[:, :-1, :].transpose(1, 2)``
    against ``input_ids[:, 1:]``) and its gradient with respect to the whole logits: the
    view's gradient in positions 0..S-2 and zero in the last position (the slice's
    backward)."""

    loss, grad_view = forward_backward(
        logits[:, :-1, :].transpose(1, 2), input_ids[:, 1:], ignore_index, compute
    )
    grad = torch.zeros(logits.shape, dtype=compute, device=logits.device)
    grad[:, :-1, :] = grad_view.transpose(1, 2)
    return loss, grad
