"""Headline benchmark: ResNet-18 fp32 batch 32 img/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-dropin]

A step is one forward pass of the seeded ResNet-18 (configs[2] of
BN folded, [32,3,224,224] -> [32,1000]) through the gfx950
HipDevice rows, with weights and the input already resident in HBM. The
runner (nert_amd.runner.Program) first fuses each Conv -> [Add] -> [Relu]
chain into one FusedConv row (bias, residual and Relu in the conv epilogue,
bit-identical outputs), pairs each stage's 3x3/2 conv with its 1x1/2
downsampling shortcut (one launch computes both; the shortcut's sums run in
another order, within the parity bar) and turns the Flatten into a view,
leaving 20 of the 49 rows; they are captured once into a HIP graph and
replayed. K replays are
timed with HIP events on the layer stream, bracketed by stream syncs. The
step's logits must match the reference executor's (the committed fixture
tests/golden/models/resnet18_bs32.npz, all 32 images, and the live
cpu_baseline run) within rel 2e-4, or the run exits 1.

Extra keys on the one JSON line:
  roofline      the Conv rows (implicit GEMM on fp32 MFMA), the dominant
                kernel family: algorithmic flops per step / summed Conv-row
                device time per step. Each Conv row's time is taken as the
                step sees it: 20 back-to-back launches of that row captured
                into one HIP graph, timed between HIP events on the layer
                stream (kernel time plus the in-graph dispatch gaps, no host
                launch overhead). Their sum must stay below ms_per_step.
  dropin        the seam as a NERT user drives it: the reference executor
                nert::Model(graph, dims, nert::HipDevice()).RunTyped (host
                input in, host logits out, 49 unfused rows launched one by
                one), wall time per call; and the device time of those 49
                unfused rows replayed as a HIP graph (no fusion, no views).
  dropin_bs1    the reference's own full-model HIP gate
                (tools/hip_model_check.cpp:57-88) on this device: ResNet-18 at
                batch 1, Model construction ms, then Run 1 and Run 2 wall ms,
                logits against the reference executor's committed fixture.
  cpu_baseline  the reference CpuDevice executor (oracle/_ref, one core) on
                the first CPU_SAMPLE_BATCH images of the same input, timed in
                this run; its logits re-check the GPU's.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ResNet-18 fp32 img/s @bs32 on 1 MI355X; Conv/GEMM % of fp32 MFMA peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
CPU_SAMPLE_BATCH = 8
ROW_REPS = 20
PARITY_RTOL = 2e-4
FIXTURE = ROOT / "tests" / "golden" / "models" / "resnet18_bs32.npz"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def max_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    g, w = got.astype(np.float64), want.astype(np.float64)
    return float(np.max(np.abs(g - w) / (np.abs(w) + 1.0)))


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(g, x: np.ndarray, gpu_logits: np.ndarray) -> dict:
    """Reference CpuDevice on a bounded sample (first CPU_SAMPLE_BATCH images)."""
    from nert_amd.graph import to_onnx
    from oracle import ref

    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "resnet18.onnx")
        with open(path, "wb") as f:
            f.write(to_onnx(g))
        lg = ref.LoadedGraph(path)
        sample = np.ascontiguousarray(x[:CPU_SAMPLE_BATCH])
        out = np.zeros((CPU_SAMPLE_BATCH, gpu_logits.shape[1]), np.float32)
        secs = ref.model_run(lg.handle, [sample], [out])
        lg.close()
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {
        "value": round(CPU_SAMPLE_BATCH / secs, 4),
        "unit": "img/s",
        "cores": 1,
        "kind": "reference",
        "sample": f"reference CpuDevice Model::RunTyped (oracle/_ref, single-threaded) on images 0-"
                  f"{CPU_SAMPLE_BATCH - 1} of the 32 ({secs:.2f} s wall)",
        "cpu_model": cpu_model(),
        "host_logical_cpus": os.cpu_count(),
        "cpus_available": affinity,
        "logits_max_rel_err_vs_gpu": max_rel_err(gpu_logits[:CPU_SAMPLE_BATCH], out),
    }


def fixture_parity(g, inputs: dict, logits: np.ndarray) -> dict:
    """All 32 logits against the reference executor's committed outputs."""
    sys.path.insert(0, str(ROOT / "tests" / "golden"))
    import model_fixtures as fx

    src = str(FIXTURE.relative_to(ROOT))
    if not FIXTURE.exists():
        return {"source": src, "checked": False, "reason": "fixture missing"}
    if not fx.matches("resnet18_bs32", g, inputs):
        return {"source": src, "checked": False, "reason": "generator fingerprint differs"}
    (want,) = fx.outputs("resnet18_bs32")
    return {"source": src, "checked": True, "images": int(logits.shape[0]), "max_rel_err": max_rel_err(logits, want)}


def dropin_leg(g, x: np.ndarray, steps: int) -> dict:
    """The seam as a NERT user drives it, next to the device time of the
    same 49 unfused rows replayed as one HIP graph."""
    import ctypes as C

    from nert_amd import abi, device
    from nert_amd.device import Event
    from nert_amd.graph import to_onnx
    from nert_amd.runner import Program

    result: dict = {}
    lib_path = ROOT / "nert_amd" / "lib" / "libnert_seamrun.so"
    if lib_path.exists():
        L = C.CDLL(str(lib_path))
        L.nert_seam_open.restype = C.c_void_p
        L.nert_seam_open.argtypes = [C.c_char_p, C.c_int, C.c_int, C.POINTER(abi.TensorDesc), C.POINTER(C.c_int64),
                                     C.c_char_p, C.c_int]
        L.nert_seam_run.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(abi.TensorDesc), C.POINTER(C.c_double),
                                    C.c_char_p, C.c_int]
        L.nert_seam_close.argtypes = [C.c_void_p]
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "resnet18.onnx")
            Path(path).write_bytes(to_onnx(g))
            ip = abi.TensorPack(abi.host_entries([x]))
            arena = C.c_int64()
            err = C.create_string_buffer(4096)
            sess = L.nert_seam_open(path.encode(), 1, 1, ip.array, C.byref(arena), err, len(err))
            if not sess:
                raise RuntimeError(f"drop-in: {err.value.decode()}")
            out = np.zeros((x.shape[0], 1000), np.float32)
            op = abi.TensorPack(abi.host_entries([out]))
            secs = C.c_double()
            try:
                for runs in (2, steps):  # first: per-geometry choices, allocator and staging warm-up
                    rc = L.nert_seam_run(sess, runs, 1, op.array, C.byref(secs), err, len(err))
                    if rc != abi.OK:
                        raise RuntimeError(f"drop-in: {err.value.decode()}")
            finally:
                L.nert_seam_close(sess)
        result.update({
            "wall_ms_per_call": round(secs.value * 1e3, 4),
            "img_s": round(x.shape[0] / secs.value, 2),
            "arena_mib": round(arena.value / 2**20, 2),
            "path": "nert::LoadGraphFromFile -> FoldConstants(CpuDevice) -> nert::Model(graph, dims, "
                    "nert::HipDevice()).RunTyped, host input staged and host logits returned every call",
            "logits": out,
        })
    prog = Program(g, fuse=False, views=False)
    prog.set_input("input", x)
    prog.capture()
    for _ in range(3):
        prog.replay()
    device.synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(steps):
        prog.replay()
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    result.update({"unfused_rows": len(prog.graph.nodes), "unfused_device_ms_per_step": round(ms, 4),
                   "unfused_device_img_s": round(x.shape[0] / (ms / 1e3), 2)})
    prog.close()
    return result


GATE_FIXTURE = ROOT / "tests" / "golden" / "models" / "resnet18_bs1.npz"


def dropin_gate_bs1() -> dict:
    """The reference's own full-model HIP gate (tools/hip_model_check.cpp:57-88)
    on this device: ResNet-18 at batch 1, nert::Model(graph, dims,
    nert::HipDevice()) construction timed, then Run 1 and Run 2 wall times,
    and the logits against the reference executor's (committed fixture)."""
    import ctypes as C

    from nert_amd import workloads
    from nert_amd.graph import to_onnx

    lib_path = ROOT / "nert_amd" / "lib" / "libnert_seamrun.so"
    if not lib_path.exists():
        return {"checked": False, "reason": "libnert_seamrun.so not built"}
    L = C.CDLL(str(lib_path))
    L.nert_seam_gate.argtypes = [C.c_char_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                 C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_double),
                                 C.c_char_p, C.c_int]
    g, inputs = workloads.resnet18(batch=1)
    x = np.ascontiguousarray(inputs["input"])
    out = np.zeros((1, 1000), np.float32)
    construct, run1, run2 = C.c_double(), C.c_double(), C.c_double()
    err = C.create_string_buffer(4096)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "resnet18_bs1.onnx")
        Path(path).write_bytes(to_onnx(g))
        rc = L.nert_seam_gate(path.encode(), x.ctypes.data, x.size, out.ctypes.data, out.size, C.byref(construct),
                              C.byref(run1), C.byref(run2), err, len(err))
    if rc != 0:
        raise RuntimeError(f"drop-in bs1 gate: {err.value.decode()}")
    result = {
        "path": "nert::LoadGraphFromFile -> nert::Model(graph, dims, nert::HipDevice()) -> Run x2 "
                "(tools/hip_model_check.cpp:57-88)",
        "batch": 1,
        "nodes": len(g.nodes),
        "construct_ms": round(construct.value, 3),
        "run1_ms": round(run1.value, 3),
        "run2_ms": round(run2.value, 3),
        "run2_img_s": round(1e3 / run2.value, 1),
        "published_mi300x_reference_hip_ms": {"construct": 80.3, "run1": 8.60, "run2": 6.85,
                                              "source": "specs/2026-10-23-amd-devcloud/resnet-model.txt:1-3"},
    }
    sys.path.insert(0, str(ROOT / "tests" / "golden"))
    import model_fixtures as fx

    if GATE_FIXTURE.exists() and fx.matches("resnet18_bs1", g, inputs):
        (want,) = fx.outputs("resnet18_bs1")
        result["max_rel_err_vs_reference_fixture"] = max_rel_err(out, want)
        result["reference_gate_max_ratio"] = float(
            np.max(np.abs(out.astype(np.float64) - want) / (1e-3 * (1 + np.abs(want.astype(np.float64))))))
    else:
        result["max_rel_err_vs_reference_fixture"] = None
    return result


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--no-dropin", action="store_true", help="skip the drop-in (reference executor) leg")
    ap.add_argument("--ops", action="store_true",
                    help="instead of the model step: the op-level cases (nert_amd/opcases.py), one JSON line each")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with one elementwise pass over 256 MiB (read 256 MiB, write 256 MiB): the "
                         "known-size kernel that scales the FETCH_SIZE/WRITE_SIZE counters of a --pmc run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the path has no multi-GPU mode", file=sys.stderr)
        return 2
    if args.ops:
        return op_cases(args)
    batch = 32

    from nert_amd import device, workloads
    from nert_amd.device import Event
    from nert_amd.runner import Program

    device.init()
    t0 = time.time()
    g, inputs = workloads.resnet18(batch=batch)
    x = inputs["input"]
    log(f"built ResNet-18 bs{batch}: {len(g.nodes)} nodes, {g.flops() / 1e9:.2f} GFLOP/step "
        f"({time.time() - t0:.1f} s)")
    prog = Program(g)
    prog.set_input("input", x)
    log(f"arena {prog.arena_bytes / 2**20:.1f} MiB")
    prog.capture()
    for _ in range(args.warmup):
        prog.replay()
    device.synchronize()
    start, stop = Event(), Event()
    start.record()
    for _ in range(args.steps):
        prog.replay()
    stop.record()
    ms_total = start.elapsed_ms(stop)
    device.synchronize()
    ms_per_step = ms_total / args.steps
    img_s = batch * args.steps / (ms_total / 1e3)
    logits = prog.output(g.outputs[0])
    log(f"graph replay: {ms_per_step:.4f} ms/step, {img_s:.1f} img/s")

    # Dominant kernel family: the Conv rows, each timed as replayed launches.
    pg = prog.graph
    conv_idx = [i for i, n in enumerate(pg.nodes) if n.op in ("Conv", "FusedConv")]
    row_ms = prog.time_rows(conv_idx, reps=ROW_REPS)
    conv_ms = np.array([row_ms[i] for i in conv_idx])
    conv_flops = np.array([conv_row_flops(pg, i) for i in conv_idx], dtype=np.float64)
    achieved = conv_flops.sum() / (conv_ms.sum() / 1e3) / 1e12
    for i, ms, fl in zip(conv_idx, conv_ms, conv_flops):
        n = pg.nodes[i]
        log(f"  {n.op:9s} {n.name:10s} W{pg.tensors[n.inputs[1]][1]} -> {pg.tensors[n.outputs[0]][1]}: "
            f"{ms * 1e3:8.1f} us {fl / (ms / 1e3) / 1e12:6.1f} TFLOP/s")
    log(f"Conv rows {conv_ms.sum():.4f} ms of the {ms_per_step:.4f} ms step "
        f"({conv_ms.sum() / ms_per_step * 100:.1f}%), {achieved:.1f} TFLOP/s")
    consistent = conv_ms.sum() < ms_per_step

    parity = fixture_parity(g, inputs, logits)
    log(f"parity vs reference fixture: {parity}")
    prog.close()

    result = {
        "metric": METRIC,
        "value": round(img_s, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64/Box-Muller seeded weights and input, BN folded)",
        "config": {
            "workload": "configs[2] ResNet-18 forward, batch 32, [32,3,224,224] -> [32,1000], opset-17 rows",
            "batch": batch,
            "nodes": len(g.nodes),
            "rows_after_fusion": len(pg.nodes),
            "gflop_per_step": round(g.flops() / 1e9, 3),
            "launch": "nert_amd runner: HIP graph replay after Conv->Add->Relu fusion (bit-identical outputs), "
                      "each stage's 3x3/2 conv paired with its 1x1/2 shortcut in one launch, the 3x3 weights packed once "
                      "into the halo kernel's LDS order, and view aliasing; "
                      "the drop-in seam path is reported under 'dropin'",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": f"Conv rows (implicit-GEMM conv kernels, split tiles finished inside the kernel; fused "
                      f"Add/Relu epilogues; 3 rows also compute their stage's 1x1 shortcut), {len(conv_idx)} per "
                      f"step for the 20 convolutions",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": (measured_traffic() or {}).get("bytes_per_conv_row"),
            "traffic_unit": "HBM bytes per Conv row",
            "traffic_source": "profiles/conv_resnet18_bs32_traffic.json (rocprofv3 --pmc FETCH_SIZE and "
                              "WRITE_SIZE passes, scaled by the copy probe)",
            "timing": f"each Conv row: {ROW_REPS} launches captured in one HIP graph, HIP events on the layer stream",
            "conv_ms_per_step": round(float(conv_ms.sum()), 4),
            "conv_share_of_step": round(float(conv_ms.sum()) / ms_per_step, 4),
            "conv_row_avg_us": round(float(conv_ms.mean()) * 1e3, 2),
            "conv_gflop_per_step": round(float(conv_flops.sum()) / 1e9, 3),
        },
        "parity": parity,
        "dropin": None,
        "dropin_bs1": None,
        "cpu_baseline": None,
    }
    ok = consistent and (not parity.get("checked") or parity["max_rel_err"] <= PARITY_RTOL)
    if not args.no_dropin:
        log("drop-in: reference executor on HipDevice ...")
        d = dropin_leg(g, x, max(5, min(args.steps, 20)))
        if "logits" in d:
            d["logits_max_rel_err_vs_replay"] = max_rel_err(d.pop("logits"), logits)
            ok = ok and d["logits_max_rel_err_vs_replay"] <= PARITY_RTOL
        result["dropin"] = d
        log(f"drop-in: {d}")
        log("drop-in gate: ResNet-18 bs1, construct + two Runs on HipDevice ...")
        gate = dropin_gate_bs1()
        result["dropin_bs1"] = gate
        log(f"drop-in gate bs1: {gate}")
        if gate.get("max_rel_err_vs_reference_fixture") is not None:
            ok = ok and gate["max_rel_err_vs_reference_fixture"] <= PARITY_RTOL
    if not args.no_cpu:
        log(f"cpu baseline: reference CpuDevice on {CPU_SAMPLE_BATCH} images ...")
        result["cpu_baseline"] = cpu_baseline(g, x, logits)
        log(f"cpu baseline {result['cpu_baseline']['value']} img/s; "
            f"logit parity max rel {result['cpu_baseline']['logits_max_rel_err_vs_gpu']:.2e}")
        ok = ok and result["cpu_baseline"]["logits_max_rel_err_vs_gpu"] <= PARITY_RTOL
    print(json.dumps(result), flush=True)
    if args.copy_probe:
        copy_probe()
    if not consistent:
        log(f"bench.py: Conv rows ({conv_ms.sum():.4f} ms) do not fit in the step ({ms_per_step:.4f} ms)")
    if not ok:
        log("bench.py: FAILED (parity above rel 2e-4 or inconsistent timing)")
        return 1
    return 0


PEAK_HBM_GBS = 8000.0
CPU_CASE_BUDGET_S = 8.0


def op_cases(args) -> int:
    """One JSON line per op-level case: kernel time (ROW_REPS launches of the
    row captured in one HIP graph, HIP events on the layer stream), the
    roofline fraction of its algorithmic work, the reference HIP layer's
    published MI300X time, and the reference CpuDevice row timed on this
    host's core (its cpu_baseline leg, whose output also checks the GPU's)."""
    from nert_amd import device, opcases
    from nert_amd.runner import Program

    device.init()
    ok = True
    for case in opcases.CASES:
        g = case.graph()
        inputs = case.inputs()
        prog = Program(g, fuse=False, views=False)
        for n, v in inputs.items():
            prog.set_input(n, v)
        prog.run()
        outs = [prog.output(t) for t in g.outputs]
        ms = prog.time_rows([0], reps=ROW_REPS)[0]
        prog.close()
        if case.bound == "mfma":
            achieved, peak, unit = case.work / (ms / 1e3) / 1e12, PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
        else:
            achieved, peak, unit = case.work / (ms / 1e3) / 1e9, PEAK_HBM_GBS, "GB/s"
        line = {"case": case.name, "op": case.op, "source": case.source,
                "shapes": {n: list(v.shape) for n, v in inputs.items()},
                "kernel_us": round(ms * 1e3, 2), "achieved": round(achieved, 2), "unit": unit,
                "peak": peak, "frac": round(achieved / peak, 4), "bound": case.bound,
                "work": case.work, "mi300x_ref_hip_ms": case.mi300x_ms,
                "speedup_vs_mi300x_ref_hip": round(case.mi300x_ms / ms, 1) if case.mi300x_ms else None}
        if not args.no_cpu:
            line["cpu_baseline"] = op_case_cpu(case, g, inputs, outs)
            ok = ok and line["cpu_baseline"]["parity_ok"]
        print(json.dumps(line), flush=True)
    return 0 if ok else 1


def op_case_cpu(case, g, inputs: dict, gpu_outs: list) -> dict:
    """The reference CpuDevice row on the same inputs (a leading-batch sample
    when the whole case would take much longer than CPU_CASE_BUDGET_S)."""
    from oracle import ref

    names = g.nodes[0].inputs
    feeds = [inputs[n] if n in inputs else g.initializers[n] for n in names]
    out_specs = [(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
    sample = 1
    if case.op == "MatMul" and feeds[0].ndim == 3:
        sample = feeds[0].shape[0]  # batches are independent: time one, scale
        feeds = [f[:1] for f in feeds]
        out_specs = [((1,) + tuple(s[1:]), d) for s, d in out_specs]
    outs = [np.zeros(s, d) for s, d in out_specs]
    t0 = time.perf_counter()
    ref.run_node(case.op, feeds, outs, case.attrs, name=case.name)
    secs = (time.perf_counter() - t0) * sample
    worst = 0.0
    exact = True
    for got, want in zip(gpu_outs, outs):
        got = got[: want.shape[0]]
        if want.dtype == np.float32:
            d = np.abs(got.astype(np.float64) - want) / (1e-4 + 1e-4 * np.abs(want.astype(np.float64)))
            worst = max(worst, float(d.max()))
        else:
            exact = exact and bool(np.array_equal(got, want))
    return {"ms": round(secs * 1e3, 3), "cores": 1, "kind": "reference",
            "sample": "whole case" if sample == 1 else f"1 of {sample} batches, time scaled by {sample}",
            "float_max_ratio_to_1e-4_bar": round(worst, 4), "int_outputs_bit_exact": exact,
            "parity_ok": worst <= 1.0 and exact}


COPY_PROBE_FLOATS = 64 << 20


def copy_probe() -> None:
    """One Relu over 64 Mi non-negative floats: 256 MiB read, 256 MiB written."""
    from nert_amd import device

    buf = device.DeviceArray.from_host(np.ones(COPY_PROBE_FLOATS, np.float32))
    out = device.DeviceArray((COPY_PROBE_FLOATS,), np.float32)
    device.check(device.lib().nert_hip_unary(0, 0, buf.ptr, out.ptr, COPY_PROBE_FLOATS, 0.0, 0.0, None), "relu")
    device.synchronize()
    buf.close()
    out.close()


def measured_traffic() -> dict | None:
    """HBM bytes per Conv row from the committed --pmc passes, if present."""
    path = ROOT / "profiles" / "conv_resnet18_bs32_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text())


def conv_row_flops(g, idx: int) -> int:
    """2 * MACs of a Conv or FusedConv row; a paired FusedConv (W2 as its
    fifth input, two outputs) also counts its 1x1 convolution. (A seventh
    input, the packed copy of W, adds no work.)"""
    n = g.nodes[idx]
    w = g.tensors[n.inputs[1]][1]
    y = g.tensors[n.outputs[0]][1]
    flops = 2 * int(np.prod(y)) * int(np.prod(w[1:]))
    if n.op == "FusedConv" and len(n.inputs) >= 6 and n.inputs[4] and len(n.outputs) == 2:
        w2 = g.tensors[n.inputs[4]][1]
        flops += 2 * int(np.prod(g.tensors[n.outputs[1]][1])) * int(np.prod(w2[1:]))
    return flops


if __name__ == "__main__":
    sys.exit(main())
