"""GPU: the nert::HipDevice() object itself, and the reference executor's
contracts on it (tests/cpp/contract.cpp drives the C++ seam directly).

  * test/hip_device_test.cpp:23-148: the device names itself "hip", is not a
    host device, serves every first-party row, allocates nothing for sizes
    <= 0, and round-trips 1 KiB; include/nert/device.hpp:33-76 adds
    release(nullptr), 64-byte alignment, zero-byte transfers and arena
    offsets.
  * test/executor_test.cpp:375-479: initializers upload once across runs; a
    row that throws inside Model::Run releases the staged inputs, and the
    same Model then runs correctly.
  * Data-dependent rejections (Gather index out of range, int64 division by
    zero, from a staged input and from a device-computed one) throw the
    reference executor's message inside Model::Run on HipDevice, and the next
    Run of the same Model succeeds.
  * FoldConstants(g, CpuDevice()) before Model(g, dims, HipDevice())
    (src/constant_folding.cpp:108-143), as the seam's callers are told to do.
"""

import ctypes as C
import os
import tempfile
from pathlib import Path

import numpy as np
import pytest

from nert_amd import abi, graph
from nert_amd.device import has_row
from nert_amd.graph import Graph
from oracle import ref
from test_library import REFERENCE_ROWS

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
CONTRACT = ROOT / "tests" / "_build" / "libnert_contract.so"
F, I = np.float32, np.int64


def _lib():
    L = C.CDLL(str(CONTRACT))
    L.contract_device_facts.argtypes = [C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int), C.c_char_p,
                                        C.c_int]
    L.contract_find_rows.argtypes = [C.POINTER(C.c_char_p), C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    L.contract_allocator_transfer.argtypes = [C.c_char_p, C.c_int]
    td = C.POINTER(abi.TensorDesc)
    L.contract_throw_then_run.argtypes = [C.c_void_p, C.c_int, td, C.c_int, td, C.c_char_p, C.c_int,
                                          C.POINTER(C.c_int64), C.c_char_p, C.c_int]
    L.contract_reject_then_run.argtypes = [C.c_void_p, C.c_int, td, td, C.c_int, td, C.c_char_p, C.c_int]
    L.contract_fold_then_run.argtypes = [C.c_void_p, C.c_int, td, C.c_int, td, C.POINTER(C.c_int),
                                         C.POINTER(C.c_int), C.c_char_p, C.c_int]
    return L


def _load(g: Graph):
    path = os.path.join(tempfile.mkdtemp(), "m.onnx")
    Path(path).write_bytes(graph.to_onnx(g))
    return ref.LoadedGraph(path)


def _ref_outputs(g: Graph, inputs):
    lg = _load(g)
    outs = [np.zeros(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
    try:
        ref.model_run(lg.handle, inputs, outs)
    finally:
        lg.close()
    return outs


def _ref_error(g: Graph, inputs) -> str:
    lg = _load(g)
    outs = [np.zeros(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
    try:
        with pytest.raises(ref.RefError) as e:
            ref.model_run(lg.handle, inputs, outs)
    finally:
        lg.close()
    return e.value.message


def test_device_names_itself(gpu):
    name = C.create_string_buffer(64)
    is_host, offsets = C.c_int(-1), C.c_int(-1)
    err = C.create_string_buffer(1024)
    rc = _lib().contract_device_facts(name, 64, C.byref(is_host), C.byref(offsets), err, 1024)
    assert rc == abi.OK, err.value.decode()
    assert name.value.decode() == "hip"
    assert is_host.value == 0 and offsets.value == 1


def test_every_reference_row_resolves_through_find(gpu):
    # The runner's fused rows are not reference op types: find answers null
    # for them, as both reference tables do (src/kernels/cpu_kernels.cpp:15-93,
    # src/hip/table.cpp:95-173).
    fused = ["FusedConv", "FusedMatMul", "FusedAddLayerNorm", "FusedAttention"]
    ops = REFERENCE_ROWS + fused + ["BatchNormalization", "NoSuchOp", ""]
    arr = (C.c_char_p * len(ops))(*[o.encode() for o in ops])
    found = (C.c_int * len(ops))()
    cpu = (C.c_int * len(ops))()
    _lib().contract_find_rows(arr, len(ops), found, cpu)
    for i, op in enumerate(ops):
        assert found[i] == cpu[i], f"{op!r}: HipDevice find {found[i]} vs CpuDevice find {cpu[i]}"
    assert sum(found) == 73
    assert all(found[ops.index(op)] == 0 for op in fused)
    assert all(has_row(op) for op in fused), "the node-level entry point serves the fused rows"


def test_allocator_and_transfer_contract(gpu):
    err = C.create_string_buffer(1024)
    rc = _lib().contract_allocator_transfer(err, 1024)
    assert rc == abi.OK, err.value.decode()


def _add_relu_graph():
    g = Graph()
    x = g.add_input("x", F, (4, 8))
    c = g.add_initializer("c", np.linspace(-1, 1, 32, dtype=F).reshape(4, 8))
    a = g.add_node("Add", [x, c], [("a", F, (4, 8))], name="add")[0]
    z = g.add_node("Relu", [a], [("z", F, (4, 8))], name="relu")[0]
    g.outputs.append(z)
    return g


@pytest.mark.parametrize("throw_op", ["Add", "Relu"])
def test_throwing_row_releases_staging_then_model_runs(gpu, throw_op):
    g = _add_relu_graph()
    x = np.random.default_rng(3).standard_normal((4, 8)).astype(F)
    (want,) = _ref_outputs(g, [x])
    lg = _load(g)
    out = np.zeros((4, 8), F)
    ip = abi.TensorPack(abi.host_entries([x]))
    op = abi.TensorPack(abi.host_entries([out]))
    counts = (C.c_int64 * 20)()
    err = C.create_string_buffer(1024)
    good_runs = 3
    try:
        rc = _lib().contract_throw_then_run(lg.handle, 1, ip.array, 1, op.array, throw_op.encode(), good_runs,
                                            counts, err, 1024)
    finally:
        lg.close()
    assert rc == abi.OK, err.value.decode()
    assert err.value.decode() == f"{throw_op} (node '{throw_op.lower()}'): boom"
    built, failed, ran, gone = (list(counts[5 * k:5 * k + 5]) for k in range(4))
    # [allocate, release, live, h2d calls, h2d bytes]
    assert built[2] == 2 and built[3] == 1 and built[4] == 128, built  # arena + resident `c`, one upload
    assert failed[2] == built[2], f"the failed Run left {failed[2] - built[2]} staged buffers allocated"
    assert failed[3] == 2 and failed[4] == 256, failed                    # it staged the input once
    assert ran[2] == built[2] and ran[3] == 2 + good_runs, ran            # residents never re-uploaded
    assert ran[4] == 128 * (2 + good_runs)
    assert gone[2] == 0 and gone[0] == gone[1], gone                     # every allocation released
    assert np.array_equal(out, want)


def _gather_graph():
    g = Graph()
    idx = g.add_input("idx", I, (3,))
    data = g.add_initializer("data", np.arange(40, dtype=F).reshape(10, 4))
    y = g.add_node("Gather", [data, idx], [("y", F, (3, 4))], {"axis": 0}, name="gather")[0]
    g.outputs.append(y)
    return g


def _div_graph(device_divisor: bool):
    g = Graph()
    x = g.add_input("x", I, (5,))
    d = g.add_input("d", I, (5,))
    if device_divisor:  # computed on the device: no host shadow, the kernel flags the zero
        one = g.add_initializer("one", np.array(1, I))
        d = g.add_node("Sub", [d, one], [("d1", I, (5,))], name="sub")[0]
    y = g.add_node("Div", [x, d], [("y", I, (5,))], name="div")[0]
    g.outputs.append(y)
    return g


@pytest.mark.parametrize("case", ["gather", "div_staged", "div_device"])
def test_data_dependent_rejection_then_model_runs(gpu, case):
    if case == "gather":
        g = _gather_graph()
        bad = [np.array([0, 10, 1], I)]
        good = [np.array([9, -10, 3], I)]
    else:
        dev = case == "div_device"
        g = _div_graph(dev)
        x = np.array([7, -7, 9, 100, -3], I)
        bad = [x, np.array([2, 3, 0, 5, 1], I) + (1 if dev else 0)]
        good = [x, np.array([2, -3, 4, 7, 1], I) + (1 if dev else 0)]
    want_msg = _ref_error(g, bad)
    (want,) = _ref_outputs(g, good)
    lg = _load(g)
    out = np.zeros(want.shape, want.dtype)
    bp = abi.TensorPack(abi.host_entries(bad))
    gp = abi.TensorPack(abi.host_entries(good))
    op = abi.TensorPack(abi.host_entries([out]))
    err = C.create_string_buffer(1024)
    try:
        rc = _lib().contract_reject_then_run(lg.handle, len(bad), bp.array, gp.array, 1, op.array, err, 1024)
    finally:
        lg.close()
    assert rc == abi.OK, err.value.decode()
    assert err.value.decode() == want_msg
    assert np.array_equal(out, want)


def test_fold_constants_then_dropin(gpu):
    """A shape computed from constants (Mul, Concat of int64 initializers)
    folds on CpuDevice into an initializer; the drop-in then runs Reshape on
    it from its resident upload."""
    g = Graph()
    x = g.add_input("x", F, (2, 3, 4))
    a = g.add_initializer("a", np.array([2], I))
    b = g.add_initializer("b", np.array([3], I))
    c = g.add_initializer("c", np.array([4], I))
    m = g.add_node("Mul", [a, b], [("m", I, (1,))], name="mul")[0]
    s = g.add_node("Concat", [m, c], [("s", I, (2,))], {"axis": 0}, name="concat")[0]
    r = g.add_node("Reshape", [x, s], [("r", F, (6, 4))], name="reshape")[0]
    z = g.add_node("Relu", [r], [("z", F, (6, 4))], name="relu")[0]
    g.outputs.append(z)
    xv = np.random.default_rng(5).standard_normal((2, 3, 4)).astype(F)
    (want,) = _ref_outputs(g, [xv])
    lg = _load(g)
    out = np.zeros((6, 4), F)
    ip = abi.TensorPack(abi.host_entries([xv]))
    op = abi.TensorPack(abi.host_entries([out]))
    folded, left = C.c_int(-1), C.c_int(-1)
    err = C.create_string_buffer(1024)
    try:
        rc = _lib().contract_fold_then_run(lg.handle, 1, ip.array, 1, op.array, C.byref(folded), C.byref(left), err,
                                           1024)
    finally:
        lg.close()
    assert rc == abi.OK, err.value.decode()
    assert folded.value == 2 and left.value == 2
    assert np.array_equal(out, want)
