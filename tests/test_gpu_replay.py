"""GPU: data-dependent errors under HIP-graph replay (nert_amd.runner.Program).

Rows with data-dependent failures check on the host when the operand has a
host shadow and otherwise raise the device error word. Inside a captured
graph the second kind is deferred: Program.check_errors() must report it
after the replay, and the flag must be cleared by the report. An int64 or
bool graph input that changes after capture re-captures the program, so the
host checks run again on the new values (no stale shadow)."""

import numpy as np
import pytest

from nert_amd.device import DeviceArray, NertError, check, lib
from nert_amd.graph import Graph
from nert_amd.runner import Program

pytestmark = pytest.mark.gpu

F, I = np.float32, np.int64
DATA = np.arange(40, dtype=F).reshape(10, 4)


def _cast_gather_graph():
    """Indices computed on the device (Cast of a float input): no host shadow."""
    g = Graph()
    x = g.add_input("x", F, (3,))
    idx = g.add_node("Cast", [x], [("idx", I, (3,))], {"to": 7}, name="cast")[0]
    data = g.add_initializer("data", DATA)
    y = g.add_node("Gather", [data, idx], [("y", F, (3, 4))], {"axis": 0}, name="gather")[0]
    z = g.add_node("Relu", [y], [("z", F, (3, 4))], name="relu")[0]
    g.outputs.append(z)
    return g


def test_replayed_gather_reports_out_of_range(gpu):
    prog = Program(_cast_gather_graph())
    try:
        prog.set_input("x", np.array([0, 1, 2], F))
        prog.capture()
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("z"), DATA[[0, 1, 2]])
        prog.set_input("x", np.array([3, 12, 1], F))   # float input: same graph, index 12 is out of range
        prog.replay()
        with pytest.raises(NertError, match="index out of range"):
            prog.check_errors()
        prog.check_errors()                             # the report cleared the flag
        prog.set_input("x", np.array([9, -10, 4], F))
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("z"), DATA[[9, 0, 4]])
    finally:
        prog.close()


def test_error_raised_before_capture_is_still_reported(gpu):
    """nert_hip_capture_begin clears the device error word before a capture.
    A bit that earlier work raised without a check (here the kernel-level
    Gather entry point with an out-of-range index, which only raises the bit)
    must survive into the next check_errors, and be cleared by that report.
    The captured program has no row that checks the word eagerly."""
    data = DeviceArray.from_host(DATA)
    idx = DeviceArray.from_host(np.array([1, 12], I))
    out = DeviceArray.from_host(np.zeros((2, 4), F))
    g = Graph()
    x = g.add_input("x", F, (3,))
    g.outputs.append(g.add_node("Relu", [x], [("y", F, (3,))], name="relu")[0])
    prog = Program(g)
    try:
        check(lib().nert_hip_gather(4, data.ptr, idx.ptr, out.ptr, 1, 10, 2, 4, None), "gather")
        prog.set_input("x", np.array([-1, 0, 2], F))
        prog.capture()                                  # clears the device word before capturing
        with pytest.raises(NertError, match="index out of range"):
            prog.check_errors()
        prog.check_errors()                             # reported once
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("y"), np.array([0, 0, 2], F))
    finally:
        prog.close()
        for t in (data, idx, out):
            t.close()


def _div_graph():
    g = Graph()
    a = g.add_input("a", I, (4,))
    d = g.add_input("d", I, (4,))
    q = g.add_node("Div", [a, d], [("q", I, (4,))], name="div")[0]
    g.outputs.append(q)
    return g


def test_changed_int64_input_recaptures_with_host_checks(gpu):
    prog = Program(_div_graph())
    a = np.array([9, -9, 100, 7], I)
    try:
        prog.set_input("a", a)
        prog.set_input("d", np.array([2, 4, 7, -3], I))
        prog.capture()
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("q"), np.array([4, -2, 14, -2], I))
        # A new divisor re-captures; its host check sees the zero at once.
        with pytest.raises(NertError, match="division by zero"):
            prog.set_input("d", np.array([2, 0, 7, 1], I))
        prog.set_input("d", np.array([3, 3, -7, 7], I))
        prog.capture()
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("q"), np.array([3, -3, -14, 1], I))
    finally:
        prog.close()


def test_workspace_growth_keeps_captured_graph_valid(gpu):
    """A graph captured with a small split-K workspace stays correct after an
    eager call grows the workspace (the old buffer is retired, not freed)."""
    rng = np.random.default_rng(11)
    g = Graph()
    a = g.add_input("a", F, (16, 2048))
    b = g.add_initializer("b", rng.standard_normal((2048, 64)).astype(F))
    y = g.add_node("MatMul", [a, b], [("y", F, (16, 64))], name="mm")[0]
    g.outputs.append(y)
    av = rng.standard_normal((16, 2048)).astype(F)
    small = Program(g)
    try:
        small.set_input("a", av)
        small.capture()
        small.replay()
        first = small.output("y")
        # A much larger skinny product on the eager path grows the shared workspace.
        g2 = Graph()
        a2 = g2.add_input("a", F, (32, 16384))
        b2 = g2.add_initializer("b", rng.standard_normal((16384, 1024)).astype(F))
        y2 = g2.add_node("MatMul", [a2, b2], [("y", F, (32, 1024))], name="mm2")[0]
        g2.outputs.append(y2)
        big = Program(g2)
        big.set_input("a", rng.standard_normal((32, 16384)).astype(F))
        big.run()
        big.output("y")
        small.replay()
        assert np.array_equal(small.output("y"), first)
        want = av.astype(np.float64) @ g.initializers["b"].astype(np.float64)
        assert np.allclose(first, want, rtol=1e-4, atol=1e-4)
    finally:
        small.close()
