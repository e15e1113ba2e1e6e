"""CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package is a from-scratch CPU restatement (numpy, plus a small C library under ``oracle/c``) of the
reference's pure-PyTorch oracles and packed-weight layouts.  It exists only to check the HIP product path.

Who may use it: ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.  Nothing
under ``forge-llm_amd/`` imports it; the product raises when its HIP library is missing instead of falling back.

Restated reference functions (every function cites the reference ``file:line`` it follows):

* ``oracle.w4``    -- ``forge/kernels/layouts/w4.py`` + ``bits.py`` + ``layout.py`` (portable_row W4 layout)
* ``oracle.gemm``  -- ``forge/kernels/ref/gemm_w4a16.py``, ``gemm_fp8.py``, ``gemm_int8.py``, ``gemm_common.py``
* ``oracle.c``     -- ``oracle/c/oracle.c`` (the same W4 dequant GEMV and exact INT8 GEMM in plain C, via ctypes)

How each function is pinned (no golden vectors for this path exist in the reference, so the checks are
closed forms, brute force, library routines and the reference tests' known answers) is listed in the header
of each module; ``tests/test_oracle_pinned.py`` holds the checks.
"""
