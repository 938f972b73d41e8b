"""CPU oracle for the fused Qwen3 SwiGLU MLP path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic the GPU library must reproduce:

* ``oracle.bf16``   -- bfloat16 bit helpers (round-to-nearest-even, ties-away variant).
* ``oracle.bfp8``   -- the bfp8 block-float weight format: 16 consecutive K values share one
  8-bit exponent, each value is 1 sign + 7 magnitude bits (numpy restatement).
* ``oracle.mlp``    -- the fp32 SwiGLU formula ``x + down(silu(gate(x)) * up(x))``.
* ``oracle.c_oracle`` -- ctypes binding of ``bfp8_ref.c``, an independent plain-C restatement of
  the quantiser, dequantiser and SwiGLU used to cross-check the numpy code.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
this package, and only to check results against.  The product (the HIP library and its Python host module)
never routes through it; it fails loudly when its native extension is missing.

Pinning (what checks each function, see ``tests/test_oracle.py``):

* bf16 rounding: every finite bf16 bin x five tails against the ties-away/RNE identity of the
  reference's ``scripts/ci/test_mlp_rounding_policy.py:16-27`` and against torch's own cast.
* SiLU*mul rounding: the reference's double-rounding known-answer pair
  (``scripts/ci/test_mlp_c1e_pack.py:533-540``) and its >25 % statistic (``:524-530``).
* bfp8 quantiser: the reference's block-float representability invariant
  (``scripts/ci/ordered_cache_hw_plan.py:243-260``), exact round trip on representable inputs,
  brute-force nearest search on single groups, the half-step error bound, and C-vs-numpy
  bit equality.
* SwiGLU formula: pure-Python float64 brute force on tiny shapes, zero input, power-of-two
  linearity in the down weight, intermediate-dimension permutation invariance, and a float64
  torch ``silu`` restatement.
"""
