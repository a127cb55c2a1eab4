"""ORACLE -- test infrastructure, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or,
for the baseline, as the timed CPU restatement of the reference torch path).
The product path (``teamredbench_amd``) never imports, calls or links it.

Contents:
  * :mod:`oracle.reference_path` -- CPU restatement of the reference torch
    backend for the stream and GEMM benchmarks (src/teamredbench/benchmarks/
    hbm.py:29-39, mfu.py:229-238), the seeded input generators of the
    benchmark configurations, fp8 per-tensor quantisation, and the parity
    comparators (ulp distance, relative Frobenius error).
  * :mod:`oracle.clib` -- ctypes binding of ``oracle/liboracle.so``, the
    plain-C restatement of the stream arithmetic and element codecs
    (stream_oracle.c) and of the reference GEMM parity harness's input
    generator (parity_inputs.cpp).

How each function is pinned (so a plausible mistake fails a check) is
listed in tests/test_oracle.py; every function there has at least one check
that does not merely retype its formula.
"""
