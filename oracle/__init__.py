"""CPU oracle for the ratchet-linear hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's ratchet-linear
path (LoomNode/local-ai-training, ``src/local_ai_training/ratchet.py`` and
``src/local_ai_training/int8_matmul.py``) so that the HIP kernels can be checked
bit-for-bit on identical inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from here, and only to check results or as the
timed CPU baseline. The product package (``local-ai-training_amd/``) never
imports, links or executes this code and has no CPU fallback.

Pinning (what fixes each function independently of this restatement):

* ``philox``     — Random123 Philox4x32-10 known-answer vectors (Salmon et al.,
                   SC'11) and the closed-form ends of Triton's int32→[0,1) map.
* ``quant``      — torch's own tensor formula (the reference's test oracle,
                   ``int8_matmul.py:225-248``) on CPU, bit-exact, including ties.
* ``gemm``       — exact float64 BLAS matmul of small integers plus torch's
                   ``((lhs.float() @ rhs.float()) * ls * rs).to(bf16)`` formula
                   (``tests/test_int8_matmul.py:181-187``).
* ``update``     — the reference's known-answer tests (``tests/test_ratchet.py``
                   17-22, 54-78, 183-193, 224-233) and its golden 60-step vector
                   (196-208, seed 1234).
* ``embedding``  — torch's own CPU embedding backward, bit-exact on integer-valued
                   gradients (every order gives the same sums); the fixed summation order
                   of the HIP kernels is restated in the function.
* ``update.row_sumsq`` — the reduction order is the HIP kernel's fixed one
                   (documented in the function); it is pinned exactly on inputs whose partial
                   sums are all representable (order-free) and by tolerance
                   against float64 elsewhere.
"""
