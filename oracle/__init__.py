"""CPU oracle for the dense hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or, in bench.py, as the timed CPU
baseline).  The product path (triton-metal_amd/) never imports it and has no
CPU fallback.

Contents
  generators.py  the reference's deterministic input formulas
  reference.py   numpy fp64 restatement of GEMM, FA forward (O, log2 LSE) and
                 FA backward (Delta, dQ, dK, dV), plus the causal extension
  native.py      ctypes loader for attn_ref.c, an independent fp64 loop
                 restatement of the same maths (built by oracle/Makefile)
  tolerance.py   the reference's error metrics and summation bound

Pinning (what checks the oracle itself; tests/test_oracle.py):
  - GEMM: exact known answers — the reference's matrix() inputs make every
    product and partial sum exactly representable, so C is exact; plus the
    C loop vs numpy.
  - FA forward/backward: the numpy restatement vs the independent C loop;
    central finite differences of sum(O*dO) (AttentionBackwardTests.swift:397-482);
    row sums of P equal 1 and O within the range of V (AttentionTests.swift:161-177);
    the reference's published training-run numbers (docs/USAGE.md:163-165:
    step-0 loss 1541.733643, |dQ| 1.4582, |dK| 1.4173, |dV| 8.3391, step-8
    loss 1482.859741).
  - Causal: the causal oracle equals the non-causal oracle applied row by row
    to each query's key prefix, and FD checks run on it too.
"""
