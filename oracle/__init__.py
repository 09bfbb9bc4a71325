"""CPU oracle for the gfx950 device layer -- TEST INFRASTRUCTURE ONLY.

Two oracles live here:
  * oracle/_ref/libnert_ref.so + libnert_refshim.so: the reference NERT CPU
    library compiled unmodified from its own sources by oracle/Makefile, with a
    C shim to run single rows (CpuDevice) or whole graphs (Model + CpuDevice).
  * oracle/restate.py: a numpy restatement of the MFMA-bound rows (Gemm,
    MatMul, Conv) in double accumulation, pinned by tests/test_oracle.py
    against the reference's known-answer literals (tests/golden/), against
    libnert_ref.so and against a brute-force loop; it checks the full-size
    cases the reference's naive loops cannot finish in seconds.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
anything from this package; the product (nert_amd/) never does.
"""
