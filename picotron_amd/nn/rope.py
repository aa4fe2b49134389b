"""Rotary position embeddings with the reference's call surface (src/picotron/nn/rope.py).

``rotary_cos_sin`` and ``apply_rotary_embedding`` restate the reference functions
(interleaved pairs on a ``(batch, heads, seq, head_dim)`` view).  ``RotaryEmbedding``
keeps the reference constructor and ``forward(query, key)``; with ``use_triton_rope`` it
rotates query and key with one fused HIP launch (autograd included) using fp32 angle
tables cached per device (grown to the longest sequence seen), and warns once and falls
back otherwise.

The reference implements only the interleaved layout.  ``layout="rotate_half"`` (pairs
``(i, i + head_dim/2)``, the Llama/HF convention) is an addition; both layouts share the
same angle table.
"""

from __future__ import annotations

import warnings

import torch
from torch import Tensor, nn

from picotron_amd.nn.triton_kernels.rope import triton_apply_rotary_embedding_pair

LAYOUTS = ("interleaved", "rotate_half")


def rotary_cos_sin(
    sequence_length: int,
    head_dim: int,
    theta: float,
    *,
    device: torch.device,
    dtype: torch.dtype,
) -> tuple[Tensor, Tensor]:
    """Cosine and sine tables ``[sequence_length, head_dim/2]`` (reference rope.py:13-32)."""

    if head_dim % 2 != 0:
        raise ValueError("RoPE requires an even attention head dimension.")
    if theta <= 0:
        raise ValueError("rope_theta must be positive.")
    inverse_frequencies = 1.0 / (
        theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim)
    )
    positions = torch.arange(sequence_length, device=device, dtype=torch.float32)
    angles = torch.outer(positions, inverse_frequencies)
    return angles.cos().to(dtype=dtype), angles.sin().to(dtype=dtype)


def apply_rotary_embedding(states: Tensor, cosine: Tensor, sine: Tensor) -> Tensor:
    """Interleaved-pair rotation of ``(batch, heads, seq, head_dim)`` states
    (reference rope.py:35-51)."""

    if states.size(-1) != cosine.size(-1) * 2:
        raise ValueError("RoPE table dimension does not match the attention head dimension.")
    cosine = cosine.unsqueeze(0).unsqueeze(0)
    sine = sine.unsqueeze(0).unsqueeze(0)
    even_states = states[..., 0::2]
    odd_states = states[..., 1::2]
    rotated = torch.stack(
        (
            even_states * cosine - odd_states * sine,
            even_states * sine + odd_states * cosine,
        ),
        dim=-1,
    )
    return rotated.flatten(start_dim=-2)


def apply_rotary_embedding_rotate_half(states: Tensor, cosine: Tensor, sine: Tensor) -> Tensor:
    """Rotate-half rotation: pairs (i, i + head_dim/2) with the same angle table."""

    if states.size(-1) != cosine.size(-1) * 2:
        raise ValueError("RoPE table dimension does not match the attention head dimension.")
    half = states.size(-1) // 2
    cosine = cosine.unsqueeze(0).unsqueeze(0)
    sine = sine.unsqueeze(0).unsqueeze(0)
    first, second = states[..., :half], states[..., half:]
    return torch.cat((first * cosine - second * sine, first * sine + second * cosine), dim=-1)


class RotaryEmbedding(nn.Module):
    """Apply RoPE to attention query and key tensors."""

    def __init__(
        self,
        head_dim: int,
        theta: float = 10_000.0,
        *,
        use_triton_rope: bool = False,
        layout: str = "interleaved",
    ) -> None:
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError("RoPE requires an even attention head dimension.")
        if theta <= 0:
            raise ValueError("rope_theta must be positive.")
        if layout not in LAYOUTS:
            raise ValueError(f"RoPE layout must be one of {LAYOUTS}.")
        self.head_dim = head_dim
        self.theta = theta
        self.layout = layout
        self.use_triton_rope = use_triton_rope
        self._triton_fallback_warned = False
        # One fp32 table pair per device, as long as the longest sequence seen: position p's
        # angles do not depend on the table length, and the kernel reads rows 0..seq-1 of a
        # longer table, so variable sequence lengths share one pair instead of one each.
        self._fp32_tables: dict[torch.device, tuple[Tensor, Tensor]] = {}

    def _tables_fp32(self, sequence_length: int, device: torch.device) -> tuple[Tensor, Tensor]:
        tables = self._fp32_tables.get(device)
        if tables is None or tables[0].size(0) < sequence_length:
            tables = rotary_cos_sin(
                sequence_length, self.head_dim, self.theta, device=device, dtype=torch.float32
            )
            self._fp32_tables[device] = tables
        return tables

    def forward(self, query: Tensor, key: Tensor) -> tuple[Tensor, Tensor]:
        """Rotate query and key using their shared sequence positions."""

        if (
            query.size(0) != key.size(0)
            or query.size(-2) != key.size(-2)
            or query.size(-1) != key.size(-1)
        ):
            raise ValueError("RoPE query and key must share batch, sequence, and head dimensions.")
        if self.use_triton_rope:
            try:
                cosine, sine = self._tables_fp32(query.size(-2), query.device)
                return triton_apply_rotary_embedding_pair(
                    query, key, cosine, sine, layout=self.layout
                )
            except Exception as error:
                if not self._triton_fallback_warned:
                    warnings.warn(
                        f"Triton RoPE unavailable; using PyTorch fallback: {error}",
                        RuntimeWarning,
                        stacklevel=2,
                    )
                    self._triton_fallback_warned = True
        cosine, sine = rotary_cos_sin(
            query.size(-2), self.head_dim, self.theta, device=query.device, dtype=query.dtype
        )
        apply = apply_rotary_embedding if self.layout == "interleaved" else apply_rotary_embedding_rotate_half
        return apply(query, cosine, sine), apply(key, cosine, sine)
