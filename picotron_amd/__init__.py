"""picotron_amd: MI355X (gfx950) HIP kernels for picotron's fused memory-bound ops.

RMSNorm and SwiGLU forward/backward, RoPE, fused cross-entropy and multi-tensor AdamW,
behind the call surface of ``picotron.nn.triton_kernels`` and the RMSNorm / SwiGLU /
RotaryEmbedding modules.  The kernels live in ``libpicotron_hip.so`` (C ABI in
``include/picotron_hip.h``), built by :mod:`picotron_amd.build`.
"""

__version__ = "0.1.0"
