"""Fused gfx950 kernels behind picotron's optional-kernel surface.

Same public names as ``picotron.nn.triton_kernels`` (reference
src/picotron/nn/triton_kernels/__init__.py:1-41); each fast path raises its
``*Unavailable`` exception when it cannot run, and the callers fall back to PyTorch.
"""

from picotron_amd.nn.triton_kernels.adamw import (
    AdamWStepWithFallback,
    FusedAdamWStepFailed,
    TritonAdamWUnavailable,
    triton_adamw_step,
    triton_clip_grad_norm_and_step,
    triton_grad_scaler_step,
    triton_unscale_and_check_,
    triton_unscale_clip_and_step,
    triton_zero_clip_grad_norm_,
)
from picotron_amd.nn.triton_kernels.attention import (
    TritonAttentionUnavailable,
    triton_causal_attention,
)
from picotron_amd.nn.triton_kernels.cross_entropy import (
    CrossEntropyWithFallback,
    TritonCrossEntropyUnavailable,
    triton_cross_entropy,
)
from picotron_amd.nn.triton_kernels.rmsnorm import (
    TritonRMSNormUnavailable,
    rms_norm_with_pytorch_forward,
    triton_residual_rms_norm,
    triton_rms_norm,
)
from picotron_amd.nn.triton_kernels.rope import (
    TritonRoPEUnavailable,
    triton_apply_rotary_embedding,
    triton_apply_rotary_embedding_pair,
)
from picotron_amd.nn.triton_kernels.swiglu import (
    TritonSwiGLUUnavailable,
    swiglu_with_pytorch_forward,
    triton_swiglu,
)

__all__ = [
    "AdamWStepWithFallback",
    "CrossEntropyWithFallback",
    "TritonAttentionUnavailable",
    "TritonAdamWUnavailable",
    "TritonCrossEntropyUnavailable",
    "TritonRMSNormUnavailable",
    "TritonRoPEUnavailable",
    "TritonSwiGLUUnavailable",
    "triton_causal_attention",
    "triton_apply_rotary_embedding",
    "triton_cross_entropy",
    "triton_rms_norm",
    "triton_swiglu",
    "swiglu_with_pytorch_forward",
    "rms_norm_with_pytorch_forward",
    # additions beyond the reference surface
    "FusedAdamWStepFailed",
    "triton_adamw_step",
    "triton_apply_rotary_embedding_pair",
    "triton_clip_grad_norm_and_step",
    "triton_grad_scaler_step",
    "triton_residual_rms_norm",
    "triton_unscale_and_check_",
    "triton_unscale_clip_and_step",
    "triton_zero_clip_grad_norm_",
]
