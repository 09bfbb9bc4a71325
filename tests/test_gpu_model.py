"""GPU end-to-end: the seeded ResNet-18 on the gfx950 layer.

Three ways to run the same ONNX model, all checked against the reference
executor on CpuDevice (oracle/_ref):
  * nert_amd.runner.Program, eager rows and HIP-graph replay (the bench path);
  * the reference's own executor nert::Model on nert::HipDevice() -- the
    drop-in: unchanged caller, new device (tests/cpp/dropin.cpp).
Logits must agree within |d| <= 2e-4 * (1 + |ref|) (north_star: rel 2e-4
end-to-end on logits). At the full batch of 32, per-image independence is
the size-independent property: images 0-1 of the batch-32 run must match the
oracle's batch-2 run of the same two images; the drop-in's batch-32 logits are
also compared, all 32 images, with the reference executor's batch-32 fixture.
"""

import ctypes as C
import os
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

from nert_amd import abi, graph, workloads
from nert_amd.runner import Program
from oracle import ref
from rowcheck import compare

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import model_fixtures as fixtures  # noqa: E402

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
DROPIN = ROOT / "tests" / "_build" / "libnert_dropin.so"
RTOL = 2e-4


@pytest.fixture(scope="module")
def resnet(gpu):
    g, inputs = workloads.resnet18(batch=32)
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "resnet18.onnx")
    Path(path).write_bytes(graph.to_onnx(g))
    lg = ref.LoadedGraph(path)
    x = inputs["input"]
    want = np.zeros((2, 1000), np.float32)
    ref.model_run(lg.handle, [np.ascontiguousarray(x[:2])], [want])
    yield g, x, lg, want
    lg.close()


def _dropin_run(lg, x, runs=2):
    L = C.CDLL(str(DROPIN))
    L.dropin_model_run.argtypes = [C.c_void_p, C.c_int, C.POINTER(abi.TensorDesc), C.c_int,
                                   C.POINTER(abi.TensorDesc), C.c_int, C.POINTER(C.c_double),
                                   C.POINTER(C.c_int64), C.c_char_p, C.c_int]
    out = np.zeros((x.shape[0], 1000), np.float32)
    ip = abi.TensorPack(abi.host_entries([x]))
    op = abi.TensorPack(abi.host_entries([out]))
    secs, arena = C.c_double(), C.c_int64()
    err = C.create_string_buffer(4096)
    rc = L.dropin_model_run(lg.handle, 1, ip.array, 1, op.array, runs, C.byref(secs), C.byref(arena), err, len(err))
    assert rc == abi.OK, err.value.decode()
    return out, secs.value, arena.value


def test_program_eager_and_graph_match_oracle(resnet):
    g, x, lg, want = resnet
    g2, _ = workloads.resnet18(batch=2)
    prog = Program(g2)
    prog.set_input("input", np.ascontiguousarray(x[:2]))
    prog.run()
    eager = prog.output("logits")
    compare(eager, want, rtol=RTOL, atol=RTOL, what="eager logits")
    prog.capture()
    for _ in range(3):
        prog.replay()
    replayed = prog.output("logits")
    assert np.array_equal(replayed, eager), "graph replay differs from eager rows"
    prog.close()


def test_batch32_images_match_oracle(resnet):
    g, x, lg, want = resnet
    prog = Program(g)
    prog.set_input("input", x)
    prog.capture()
    prog.replay()
    logits = prog.output("logits")
    assert logits.shape == (32, 1000) and np.all(np.isfinite(logits))
    compare(logits[:2], want, rtol=RTOL, atol=RTOL, what="bs32 images 0-1")
    prog.close()


def test_reference_executor_on_hipdevice(resnet):
    """nert::Model(graph, dims, HipDevice()) -- the drop-in swap."""
    g, x, lg, want = resnet
    got, secs, arena = _dropin_run(lg, np.ascontiguousarray(x[:2]))
    assert arena > 0
    compare(got, want, rtol=RTOL, atol=RTOL, what="drop-in logits")


def test_dropin_end_to_end_bs32(resnet):
    """The drop-in at the benchmark's batch: nert::Model(graph, dims,
    HipDevice()).RunTyped on all 32 images (per run: the executor's input
    staging through the seam's Transfer, every row launched eagerly, the
    blocking output copy). Images 0-1 match the oracle; the wall time per warm
    run is printed beside the device-only time of the runner's graph replay
    (the benchmark's step)."""
    g, x, lg, want = resnet
    _dropin_run(lg, x, runs=1)  # first run: per-geometry kernel choices, allocator warm-up
    got, secs, _ = _dropin_run(lg, x, runs=5)
    compare(got[:2], want, rtol=RTOL, atol=RTOL, what="drop-in bs32 logits, images 0-1")
    # All 32 images against the reference executor's own bs32 run (the
    # committed fixture, written by tests/golden/make_model_fixtures.py).
    assert fixtures.matches("resnet18_bs32", g, {"input": x}), "fixture made from another graph or input"
    (want32,) = fixtures.outputs("resnet18_bs32")
    compare(got, want32, rtol=RTOL, atol=RTOL, what="drop-in bs32 logits, all 32 images vs the reference executor")
    prog = Program(g)
    prog.set_input("input", x)
    prog.capture()
    for _ in range(5):
        prog.replay()
    from nert_amd.device import Event, synchronize
    synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(20):
        prog.replay()
    e1.record()
    device_ms = e0.elapsed_ms(e1) / 20
    compare(prog.output(g.outputs[0]), got, rtol=RTOL, atol=RTOL, what="runner vs drop-in bs32 logits")
    prog.close()
    print(f"\nModel::RunTyped on HipDevice, ResNet-18 bs32: {secs * 1e3:.3f} ms wall per run "
          f"({32 / secs:.0f} img/s, host input staged each run); runner graph replay, inputs resident: "
          f"{device_ms:.3f} ms per step ({32 / device_ms * 1e3:.0f} img/s)")


@pytest.mark.parametrize("batch", [1, 2])
def test_fused_vit_program_is_bit_identical(gpu, batch):
    """The MatMul+scale+bias+Gelu fusion, the residual Add+LayerNorm fusion
    and the view aliasing change no output bit (ViT-B/16, two layers,
    batch 1 and 2: 197 and 394 token rows; the attention fusion, which is
    not bit-exact, left out)."""
    g, inputs = workloads.vit_b16(batch=batch, layers=2)
    outs = []
    for fuse, views in ((False, False), (True, True)):
        prog = Program(g, fuse=fuse, views=views, attention=False)
        prog.set_input("input", inputs["input"])
        prog.run()
        outs.append(prog.output(g.outputs[0]))
        prog.close()
    fused = Program(g, attention=False).graph.nodes
    assert sum(1 for n in fused if n.op == "FusedMatMul") == 10
    # At batch 1 the position-embedding Add has same-shape operands too, so
    # the first LayerNorm fuses with it as well.
    assert sum(1 for n in fused if n.op == "FusedAddLayerNorm") == (5 if batch == 1 else 4)
    assert np.array_equal(outs[0], outs[1])


def test_fused_detector_program_is_bit_identical(gpu):
    """The Conv -> Sigmoid -> Mul (SiLU) fusion changes no output bit: the
    detector's sigmoid scores, top scores, boxes and classes (batch 1,
    128x128) from the fused program equal the separate rows'."""
    g, inputs = workloads.detector(batch=1, size=128, k=50, expose_scores=True)
    outs = []
    for fuse, views in ((False, False), (True, True)):
        prog = Program(g, fuse=fuse, views=views)
        try:
            if fuse:
                assert sum(1 for n in prog.graph.nodes if n.attrs.get("activation") == "Silu") == 7
            prog.set_input("input", inputs["input"])
            prog.run()
            prog.check_errors()
            outs.append([prog.output(t) for t in g.outputs])
        finally:
            prog.close()
    for a, b in zip(*outs):
        assert a.dtype == b.dtype and np.array_equal(a, b)


def test_fused_attention_program_matches_separate_rows(gpu):
    """With the attention blocks fused (FusedAttention, one kernel for QK^T,
    scale, Softmax and PV), the ViT logits stay within the 2e-4 bar of the
    separate rows and of the reference executor (ViT-B/16, two layers,
    batch 2)."""
    g, inputs = workloads.vit_b16(batch=2, layers=2)
    fused = Program(g)
    try:
        assert sum(1 for n in fused.graph.nodes if n.op == "FusedAttention") == 2
        assert sum(1 for n in fused.graph.nodes if n.op == "FusedMatMul") == 8
        fused.set_input("input", inputs["input"])
        fused.run()
        fused.check_errors()
        got = fused.output(g.outputs[0])
    finally:
        fused.close()
    plain = Program(g, fuse=False, views=False)
    try:
        plain.set_input("input", inputs["input"])
        plain.run()
        want = plain.output(g.outputs[0])
    finally:
        plain.close()
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "vit2.onnx")
    Path(path).write_bytes(graph.to_onnx(g))
    lg = ref.LoadedGraph(path)
    try:
        oracle = np.zeros(got.shape, np.float32)
        ref.model_run(lg.handle, [inputs["input"]], [oracle])
    finally:
        lg.close()
    compare(got, want, rtol=RTOL, atol=RTOL, what="fused vs separate rows")
    compare(got, oracle, rtol=RTOL, atol=RTOL, what="fused vs reference executor")


def test_fused_program_is_bit_identical(gpu):
    """The runner's Conv+Add+Relu fusion changes no output bit (batch 2);
    pairing each stage's 3x3/2 conv with its 1x1/2 shortcut in one launch
    changes only the order of the shortcut's additions, so the logits stay
    within the end-to-end bar of the unpaired program's."""
    g, inputs = workloads.resnet18(batch=2)
    outs = []
    for fuse, pairs in ((False, False), (True, False), (True, True)):
        prog = Program(g, fuse=fuse, pairs=pairs)
        if pairs:
            assert sum(1 for n in prog.graph.nodes if len(n.outputs) == 2 and n.op == "FusedConv") == 3
        prog.set_input("input", inputs["input"])
        prog.run()
        outs.append(prog.output(g.outputs[0]))
        prog.close()
    assert np.array_equal(outs[0], outs[1])
    compare(outs[2], outs[1], rtol=2e-4, atol=2e-4, what="paired vs unpaired program")


def test_reference_model_gate_bs1(gpu, tmp_path):
    """The reference's full-model HIP gate (tools/hip_model_check.cpp:57-88)
    through the seam: ResNet-18 at batch 1, nert::Model on HipDevice() built,
    then Run twice; run 2's logits against the reference executor's batch-1
    fixture within rel 2e-4 (the gate's own bar is 1e-3 * (1 + |ref|))."""
    g, inputs = workloads.resnet18(batch=1)
    assert fixtures.matches("resnet18_bs1", g, inputs), "fixture made from another graph or input"
    (want,) = fixtures.outputs("resnet18_bs1")
    L = C.CDLL(str(ROOT / "nert_amd" / "lib" / "libnert_seamrun.so"))
    L.nert_seam_gate.argtypes = [C.c_char_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                 C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_double),
                                 C.c_char_p, C.c_int]
    path = str(tmp_path / "resnet18_bs1.onnx")
    Path(path).write_bytes(graph.to_onnx(g))
    x = np.ascontiguousarray(inputs["input"])
    out = np.zeros((1, 1000), np.float32)
    times = [C.c_double() for _ in range(3)]
    err = C.create_string_buffer(4096)
    rc = L.nert_seam_gate(path.encode(), x.ctypes.data, x.size, out.ctypes.data, out.size,
                          *(C.byref(t) for t in times), err, len(err))
    assert rc == abi.OK, err.value.decode()
    compare(out, want, rtol=RTOL, atol=RTOL, what="gate logits, ResNet-18 bs1")
    print(f"\nResNet-18 bs1 gate on HipDevice: construct {times[0].value:.1f} ms, run 1 {times[1].value:.2f} ms, "
          f"run 2 {times[2].value:.2f} ms")
