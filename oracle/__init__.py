"""CPU oracle for the NanoQuant binary low-rank inference path.

TEST INFRASTRUCTURE ONLY. This package is the checker: it may be imported by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and by nothing else. The product (``nanoquant_amd``) never imports,
links or calls it, and no result of the product is ever produced by it.

It restates, on the CPU, the reference algorithms of the path:

* ``pack_binary_gemv`` / ``unpack_binary_gemv`` (reference
  ``src/nanoquant/kernel/utils.py:51-183``),
* ``pack_binary_marlin`` / ``pack_binary_marlin_fused`` (``kernel/utils.py:186-284``),
* the dequantize-and-matmul forward of ``NanoQuantLinear._compute_forward``
  (``src/nanoquant/modules/linear.py:282-291``) in float64 (the parity truth) and in
  the reference's own torch-CPU form (the timed CPU baseline),
* the op-level shape/argument rules of ``nanoquant_dyn_forward``
  (``kernel/cuda/gemv_kernel.cu:308-346``) and ``marlin_onebit_forward``
  (``kernel/cuda/gemm.cpp:36-56``).

How each function is pinned is stated in its docstring; ``tests/test_oracle.py``
holds the pins.
"""
from .nq_oracle import *  # noqa: F401,F403
