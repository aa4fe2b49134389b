"""Attention entry point of picotron's fused-kernel surface, kept for import compatibility.

The reference's ``triton_causal_attention`` (src/picotron/nn/triton_kernels/attention.py)
is an fp16 inference-only flash-attention forward: a dense contraction, outside this
library's memory-bound kernel set.  Here it always raises
:class:`TritonAttentionUnavailable`, which the reference's callers already treat as "use
the PyTorch attention path".
"""

from __future__ import annotations

from torch import Tensor


class TritonAttentionUnavailable(RuntimeError):
    """Raised because fused attention is not part of this kernel library."""


def triton_causal_attention(
    query: Tensor, key: Tensor, value: Tensor, *, sliding_window_size: int | None = None
) -> Tensor:
    del query, key, value, sliding_window_size
    raise TritonAttentionUnavailable(
        "Fused causal attention is not implemented by the HIP kernel library; "
        "use the PyTorch attention path."
    )
