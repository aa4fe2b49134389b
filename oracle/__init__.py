"""Oracle: a CPU-checkable restatement of the reference algorithms (TEST INFRASTRUCTURE).

This package is what the tests compare against, not the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it;
nothing in ``picotron_amd`` does.  Each function restates AndyMLAndAI/picotron's PyTorch
path for one op and cites the reference file:line it follows:

  rmsnorm        src/picotron/nn/triton_kernels/rmsnorm.py:49-60, 96-134
  swiglu         src/picotron/nn/triton_kernels/swiglu.py:59-81; src/picotron/nn/feedforward.py:26-43
  rope           src/picotron/nn/rope.py:13-51 (+ the rotate-half layout, no reference code)
  cross_entropy  src/picotron/nn/triton_kernels/cross_entropy.py:97-109 (F.cross_entropy)
  adamw          src/picotron/nn/triton_kernels/adamw.py:34-47 -> torch.optim.AdamW
                 (src/picotron/training/train_loop.py:308-325)

The functions are written in torch so the same code runs on CPU tensors (small cases,
golden fixtures) and on GPU tensors (full-size parity in fp64/fp32, executed by torch's own
kernels, never by the HIP library).  ``compute`` selects the arithmetic dtype (fp64 by
default).  ``fallback_*`` functions run the reference's PyTorch fallback exactly as the
reference executes it (input dtypes, op order), for the CPU baseline and the fp32 parity
target.

Pinning (tests/test_oracle.py): every function is checked against something other than
its own formula -- the reference's known-answer tests (CE mean 1.2887259920, AdamW 0.899),
torch library routines (autograd of the forward, ``torch.autograd.gradcheck``,
``F.silu``, ``F.cross_entropy``, ``torch.optim.AdamW``), closed forms and invariants.
No function is "parity unpinned".
"""
