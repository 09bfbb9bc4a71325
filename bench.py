"""Headline benchmark: ResNet-18 fp32 batch 32 img/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one forward pass of the seeded ResNet-18 (configs[2] of
BN folded, [32,3,224,224] -> [32,1000]) through the gfx950
HipDevice rows, with weights and the input already resident in HBM. The
runner first fuses each Conv -> [Add] -> [Relu] chain into one FusedConv row
(bias, residual and Relu in the conv epilogue, bit-identical outputs) and
turns the Flatten into a view of its input, which leaves 23 rows out of 49;
they are captured once into a HIP graph and replayed. K replays are timed with HIP events on the layer stream, bracketed
by stream syncs.

Extra keys on the one JSON line:
  roofline      the Conv rows (implicit GEMM on fp32 MFMA), the dominant
                kernel: algorithmic flops per step / summed Conv duration per
                step, both from HIP events around every Conv row on the layer
                stream, against the 157.3 TFLOP/s fp32 matrix peak.
  cpu_baseline  the reference CpuDevice executor (oracle/_ref, one core) on
                the first 4 images of the same input, timed in this run; its
                logits also re-check the GPU logits for those images.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ResNet-18 fp32 img/s @bs32 on 1 MI355X; Conv/GEMM % of fp32 MFMA peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
CPU_SAMPLE_BATCH = 4


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


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
    want = out.astype(np.float64)
    got = gpu_logits[:CPU_SAMPLE_BATCH].astype(np.float64)
    rel = float(np.max(np.abs(got - want) / (np.abs(want) + 1.0)))
    return {
        "value": round(CPU_SAMPLE_BATCH / secs, 4),
        "unit": "img/s",
        "cores": 1,
        "kind": "reference",
        "sample": f"reference CpuDevice Model::RunTyped on {CPU_SAMPLE_BATCH} of the 32 images "
                  f"({secs:.2f} s wall, single-threaded); host has {os.cpu_count()} logical CPUs",
        "logits_max_rel_err_vs_gpu": rel,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--eager", action="store_true", help="time per-row launches instead of graph replay")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with one elementwise pass over 256 MiB (read 256 MiB, write 256 MiB): the "
                         "known-size kernel that scales the FETCH_SIZE/WRITE_SIZE counters of a --pmc run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the path has no multi-GPU mode", file=sys.stderr)
        return 2

    from nert_amd import device, workloads
    from nert_amd.device import Event
    from nert_amd.runner import Program

    device.init()
    t0 = time.time()
    g, inputs = workloads.resnet18(batch=args.batch)
    x = inputs["input"]
    log(f"built ResNet-18 bs{args.batch}: {len(g.nodes)} nodes, {g.flops() / 1e9:.2f} GFLOP/step "
        f"({time.time() - t0:.1f} s)")
    prog = Program(g)
    prog.set_input("input", x)
    log(f"arena {prog.arena_bytes / 2**20:.1f} MiB")

    if args.eager:
        step = prog.run
    else:
        prog.capture()
        step = prog.replay
    for _ in range(args.warmup):
        step()
    device.synchronize()
    start, stop = Event(), Event()
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    ms_total = start.elapsed_ms(stop)
    device.synchronize()
    ms_per_step = ms_total / args.steps
    img_s = args.batch * args.steps / (ms_total / 1e3)
    logits = prog.output(g.outputs[0])
    log(f"{'eager' if args.eager else 'graph'}: {ms_per_step:.3f} ms/step, {img_s:.1f} img/s")

    # Roofline of the dominant kernel family (Conv rows, fused or not),
    # events per row.
    pg = prog.graph
    conv_ops = {"Conv", "FusedConv"}
    conv_idx = [i for i, n in enumerate(pg.nodes) if n.op in conv_ops]
    reps = 5
    conv_ms = np.zeros(len(conv_idx))
    for _ in range(reps):
        t = prog.run_timed(conv_ops)
        conv_ms += np.array([t[i] for i in conv_idx])
    conv_ms /= reps
    device.synchronize()
    conv_flops = np.array([Graph_flops(pg, i) for i in conv_idx], dtype=np.float64)
    achieved = conv_flops.sum() / (conv_ms.sum() / 1e3) / 1e12
    for i, ms, fl in zip(conv_idx, conv_ms, conv_flops):
        n = pg.nodes[i]
        log(f"  {n.op:9s} {n.name:10s} W{pg.tensors[n.inputs[1]][1]} -> {pg.tensors[n.outputs[0]][1]}: "
            f"{ms * 1e3:8.1f} us {fl / (ms / 1e3) / 1e12:6.1f} TFLOP/s")
    log(f"Conv total {conv_ms.sum():.3f} ms/step ({conv_ms.sum() / ms_per_step * 100:.0f}% of step), "
        f"{achieved:.1f} TFLOP/s")

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
            "batch": args.batch,
            "nodes": len(g.nodes),
            "rows_after_fusion": len(pg.nodes),
            "gflop_per_step": round(g.flops() / 1e9, 3),
            "launch": ("eager rows" if args.eager else "HIP graph replay") +
                      " after Conv->Add->Relu fusion (bit-identical outputs) and view aliasing",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "Conv rows (implicit-GEMM conv kernels + split-K reduce; 17 of 20 carry the fused "
                      "Add/Relu epilogue), 20 per step",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": (measured_traffic() or {}).get("bytes_per_conv_row"),
            "traffic_unit": "HBM bytes per Conv row",
            "traffic_source": "profiles/conv_resnet18_bs32_traffic.json (rocprofv3 --pmc FETCH_SIZE and "
                              "WRITE_SIZE passes, scaled by the copy probe)",
            "conv_ms_per_step": round(float(conv_ms.sum()), 4),
            "conv_launch_avg_us": round(float(conv_ms.mean()) * 1e3, 2),
            "conv_gflop_per_step": round(float(conv_flops.sum()) / 1e9, 3),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("cpu baseline: reference CpuDevice on 4 images ...")
        result["cpu_baseline"] = cpu_baseline(g, x, logits)
        log(f"cpu baseline {result['cpu_baseline']['value']} img/s; "
            f"logit parity max rel {result['cpu_baseline']['logits_max_rel_err_vs_gpu']:.2e}")
    print(json.dumps(result), flush=True)
    prog.close()
    if args.copy_probe:
        copy_probe()
    return 0


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


def Graph_flops(g, idx: int) -> int:
    n = g.nodes[idx]
    w = g.tensors[n.inputs[1]][1]
    y = g.tensors[n.outputs[0]][1]
    return 2 * int(np.prod(y)) * int(np.prod(w[1:]))


if __name__ == "__main__":
    sys.exit(main())
