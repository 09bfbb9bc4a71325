"""CPU oracle for the gfx950 device layer -- TEST INFRASTRUCTURE ONLY.

Two oracles live here:
  * oracle/_ref/libnert_ref.so + libnert_refshim.so: the reference NERT CPU
    library compiled unmodified from its own sources by oracle/Makefile, with a
    C shim to run single rows (CpuDevice) or whole graphs (Model + CpuDevice).
  * oracle/nert_oracle.c (-> oracle/_ref/libnert_oracle.so): a plain-C
    restatement of the hot-path rows, pinned against the reference's golden
    vectors and against libnert_ref.so by tests/.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
anything from this package; the product (nert_amd/) never does.
"""
