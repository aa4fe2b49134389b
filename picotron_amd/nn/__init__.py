"""Module surfaces of the fused kernels: RMSNorm, SwiGLU and RotaryEmbedding."""

from picotron_amd.nn.feedforward import SwiGLU
from picotron_amd.nn.norm import RMSNorm
from picotron_amd.nn.rope import RotaryEmbedding, apply_rotary_embedding, rotary_cos_sin

__all__ = ["RMSNorm", "RotaryEmbedding", "SwiGLU", "apply_rotary_embedding", "rotary_cos_sin"]
