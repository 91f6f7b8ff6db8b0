"""CPU oracle for the fused QLoRA hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what each hot-path operator of the reference
(fokyso82002-rgb/rus, ``solution/kernels.py`` and ``solution/ops.py``) computes:

* ``oracle.ops``   — NF4 double-quant dequant (numpy, bit-exact fp16), residual+RMSNorm fwd/bwd,
  LoRA+NeoX RoPE fwd/bwd, SwiGLU fwd/bwd and the chunked lm_head cross-entropy (eager torch on
  the CPU, fp32 arithmetic with the reference's casts);
* ``oracle.stack`` — the packed Qwen2 decoder stack with LoRA on q/v, as an eager fp32 autograd
  composition.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker or the timed CPU baseline. The product (``rus_amd``) never imports it
and has no CPU fallback.

How each function is pinned (beyond restating the reference's formula) is listed in the
docstring of the function and checked by ``tests/test_oracle.py``.
"""
