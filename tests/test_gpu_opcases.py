"""GPU parity of the op-level measurement cases (nert_amd/opcases.py: the
reference's published op-bench fixtures, bench/runtime/main.cpp:331-674,
and BASELINE.json configs[0]/configs[1]) at their full sizes, through the
runner the bench times them with.

The reference CpuDevice row is the oracle wherever it finishes in seconds;
configs[1](a) and (b) (17 GFLOP each, a minute of the reference's naive
loops) are checked against the numpy restatement (oracle/restate.py: double
accumulation, one rounding), which tests/test_oracle.py pins to the
reference row. Float outputs within 1e-4 + 1e-4|ref|; ArgMax bit-exact."""

import numpy as np
import pytest

from nert_amd import opcases
from nert_amd.runner import Program
from oracle import restate
from rowcheck import compare, run_ref

pytestmark = pytest.mark.gpu

RESTATED = {"cfg1a_matmul_8x1024", "cfg1b_gemm_2048x1024x4096"}


@pytest.mark.parametrize("case", opcases.CASES, ids=[c.name for c in opcases.CASES])
def test_op_case_matches_oracle(gpu, case):
    g = case.graph()
    inputs = case.inputs()
    prog = Program(g, fuse=False, views=False)
    try:
        for n, v in inputs.items():
            prog.set_input(n, v)
        prog.capture()  # as the bench times it: replayed rows
        prog.replay()
        prog.check_errors()
        got = [prog.output(t) for t in g.outputs]
    finally:
        prog.close()
    feeds = [inputs[n] if n in inputs else g.initializers[n] for n in g.nodes[0].inputs]
    if case.name in RESTATED:
        if case.op == "MatMul":
            want = [restate.matmul(*feeds)]
        else:
            want = [restate.gemm(feeds[0], feeds[1], feeds[2], trans_b=1, alpha=1.0, beta=1.0)]
    else:
        specs = [(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
        want, err = run_ref(case.op, feeds, specs, case.attrs, name=case.name)
        assert err is None, err
    for a, b, t in zip(got, want, g.outputs):
        compare(a, np.asarray(b).astype(a.dtype) if a.dtype != np.float32 else np.asarray(b, np.float32),
                what=f"{case.name} {t}")
