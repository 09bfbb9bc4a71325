"""Replays one of the seeded BASELINE workloads through the runner, for
timing and kernel traces:

    python3 -m nert_amd.replay {resnet18,vit,detector} [--runs N] [--eager] [--copy-probe]

Builds the program (Conv chain fusion, Add+LayerNorm fusion, view
aliasing), binds the seeded input, runs it once eagerly, captures it into a
HIP graph and replays it N times between HIP events on the layer stream
(--eager: N eager runs instead). Prints one line: workload, ms per replay,
and the algorithmic GFLOP of the graph. --copy-probe ends with one Relu over
256 MiB, the known-size dispatch that calibrates --pmc byte counters.

    python3 -m nert_amd.replay rows [--runs N]

Times ConvTranspose and Einsum rows at decoder / attention sizes on their
MFMA GEMM paths and on the exact double-sum paths (NERT_HIP_CONVT_EXACT=1,
NERT_HIP_EINSUM_EXACT=1): microseconds per row between HIP events, TFLOP/s,
and the largest difference between the two paths relative to the 1e-4 bar;
then InstanceNormalization and GridSample rows: microseconds and TB/s of
their algorithmic bytes (one read of X and the grid, one write of Y).

    python3 -m nert_amd.replay transfer [--runs N]

Times the blocking host<->device copies (nert_hip_memcpy_h2d/d2h) at the
workloads' input sizes -- the per-run staging the executor does
(src/executor.cpp:451-478) -- from pageable numpy memory with the pinned
bounce buffers on and off (NERT_HIP_STAGING), and from pinned memory. Prints
one line per size, direction and path: GB/s and ms per copy (median of N).
"""

from __future__ import annotations

import argparse
import sys

from . import device, workloads
from .device import Event
from .runner import Program

BUILDERS = {
    "resnet18": lambda: workloads.resnet18(batch=32),
    "vit": lambda: workloads.vit_b16(batch=16),
    "detector": lambda: workloads.detector(batch=8),
}


def _transfer(runs: int) -> None:
    import os
    import time

    import numpy as np

    from .device import DeviceArray, PinnedArray, check, lib

    sizes = {"resnet18 bs32 input": 32 * 3 * 224 * 224 * 4, "detector bs8 input": 8 * 3 * 640 * 640 * 4}
    for label, n in sizes.items():
        host = np.random.default_rng(0).integers(0, 256, n, dtype=np.uint8)
        back = np.empty_like(host)
        pinned = PinnedArray((n,), np.uint8)
        pinned.array[:] = host
        buf = DeviceArray((n,), np.uint8)
        paths = [("pageable, staged", host, back, "1"), ("pageable, plain", host, back, "0"),
                 ("pinned", pinned.array, pinned.array, "1")]
        for name, src, dst, staging in paths:
            os.environ["NERT_HIP_STAGING"] = staging
            for direction in ("h2d", "d2h"):
                times = []
                for _ in range(runs + 1):
                    t0 = time.perf_counter()
                    if direction == "h2d":
                        check(lib().nert_hip_memcpy_h2d(buf.ptr, src.ctypes.data, n), "h2d")
                    else:
                        check(lib().nert_hip_memcpy_d2h(dst.ctypes.data, buf.ptr, n), "d2h")
                    times.append(time.perf_counter() - t0)
                t = sorted(times[1:])[len(times[1:]) // 2]
                print(f"transfer {label} ({n / 2**20:.1f} MiB) {direction} {name}: "
                      f"{n / t / 1e9:.1f} GB/s, {t * 1e3:.3f} ms", flush=True)
        os.environ.pop("NERT_HIP_STAGING", None)
        buf.close()
        pinned.close()


def _rows(runs: int) -> None:
    import os

    import numpy as np

    from .graph import Graph

    rng = np.random.default_rng(0)
    cases = []
    for (b, c, h, m, k, s, p) in [(4, 64, 64, 32, 4, 2, 1), (8, 256, 32, 128, 2, 2, 0), (2, 128, 56, 64, 3, 1, 1)]:
        g = Graph()
        g.add_input("x", np.float32, (b, c, h, h))
        g.add_initializer("w", (rng.standard_normal((c, m, k, k)) * 0.05).astype(np.float32))
        g.add_initializer("bias", rng.standard_normal(m).astype(np.float32))
        o = s * (h - 1) + k - 2 * p
        g.add_node("ConvTranspose", ["x", "w", "bias"], [("y", np.float32, (b, m, o, o))],
                   {"strides": [s, s], "pads": [p, p, p, p]})
        g.outputs = ["y"]
        cases.append((f"ConvTranspose x{(b, c, h, h)} w{(c, m, k, k)} stride {s} pad {p}", g,
                       {"x": rng.standard_normal((b, c, h, h)).astype(np.float32)}, 2 * b * c * h * h * m * k * k,
                       "NERT_HIP_CONVT_EXACT"))
    for eq, sa, sb in [("bhqd,bhkd->bhqk", (16, 12, 197, 64), (16, 12, 197, 64)),
                       ("bhqk,bhkd->bhqd", (16, 12, 197, 197), (16, 12, 197, 64)),
                       ("ij,jk->ik", (1024, 1024), (1024, 1024))]:
        g = Graph()
        g.add_input("a", np.float32, sa)
        g.add_input("b", np.float32, sb)
        out = np.einsum(eq, np.zeros(sa, np.float32), np.zeros(sb, np.float32)).shape
        g.add_node("Einsum", ["a", "b"], [("y", np.float32, out)], {"equation": eq})
        g.outputs = ["y"]
        cases.append((f"Einsum {eq} {sa} {sb}", g, {"a": rng.standard_normal(sa).astype(np.float32),
                                                    "b": rng.standard_normal(sb).astype(np.float32)},
                      2 * int(np.prod(out)) * sa[-1], "NERT_HIP_EINSUM_EXACT"))

    def timed(g, inputs, env, reps):
        os.environ.update(env)
        try:
            prog = Program(g, fuse=False)
            for n in g.inputs:
                prog.set_input(n, inputs[n])
            prog.run()
            device.synchronize()
            start, stop = Event(), Event()
            start.record()
            for _ in range(reps):
                prog.run()
            stop.record()
            ms = start.elapsed_ms(stop) / reps
            out = prog.output(g.outputs[0])
            prog.close()
        finally:
            for k in env:
                os.environ.pop(k, None)
        return ms, out

    for name, g, inputs, flops, var in cases:
        ms_fast, y_fast = timed(g, inputs, {}, runs)
        ms_exact, y_exact = timed(g, inputs, {var: "1"}, max(1, runs // 5))
        ratio = float(np.max(np.abs(y_fast.astype(np.float64) - y_exact) / (1e-4 + 1e-4 * np.abs(y_exact))))
        print(f"{name}: MFMA path {ms_fast * 1e3:.1f} us ({flops / ms_fast / 1e9:.1f} TFLOP/s), exact path "
              f"{ms_exact * 1e3:.1f} us ({flops / ms_exact / 1e9:.2f} TFLOP/s), {ms_exact / ms_fast:.0f}x; "
              f"max |diff| / (1e-4 + 1e-4 |exact|) = {ratio:.3f}", flush=True)

    for shp in [(1, 64, 256, 256), (8, 128, 64, 64), (4, 256, 32, 32), (16, 32, 128, 128), (2, 512, 16, 16)]:
        g = Graph()
        g.add_input("x", np.float32, shp)
        g.add_initializer("s", rng.standard_normal(shp[1]).astype(np.float32))
        g.add_initializer("b", rng.standard_normal(shp[1]).astype(np.float32))
        g.add_node("InstanceNormalization", ["x", "s", "b"], [("y", np.float32, shp)], {"epsilon": 1e-5})
        g.outputs = ["y"]
        ms, _ = timed(g, {"x": rng.standard_normal(shp).astype(np.float32)}, {}, runs)
        nbytes = 8 * int(np.prod(shp))
        print(f"InstanceNormalization {shp}: {ms * 1e3:.1f} us, {nbytes / ms / 1e9:.2f} TB/s", flush=True)
    for (n, c, h, w, ho, wo) in [(1, 64, 128, 128, 128, 128), (4, 32, 64, 64, 96, 96), (8, 256, 16, 16, 32, 32)]:
        for mode, pad in [("bilinear", "zeros"), ("nearest", "border"), ("bilinear", "reflection")]:
            g = Graph()
            g.add_input("x", np.float32, (n, c, h, w))
            g.add_input("grid", np.float32, (n, ho, wo, 2))
            g.add_node("GridSample", ["x", "grid"], [("y", np.float32, (n, c, ho, wo))],
                       {"mode": mode, "padding_mode": pad, "align_corners": 0})
            g.outputs = ["y"]
            feeds = {"x": rng.standard_normal((n, c, h, w)).astype(np.float32),
                     "grid": rng.uniform(-1.1, 1.1, (n, ho, wo, 2)).astype(np.float32)}
            ms, _ = timed(g, feeds, {}, runs)
            nbytes = 4 * (n * c * h * w + n * ho * wo * 2 + n * c * ho * wo)
            print(f"GridSample {mode}/{pad} x{(n, c, h, w)} -> {ho}x{wo}: {ms * 1e3:.1f} us, "
                  f"{nbytes / ms / 1e9:.2f} TB/s", flush=True)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("workload", choices=sorted(BUILDERS) + ["rows", "transfer"])
    ap.add_argument("--runs", type=int, default=10)
    ap.add_argument("--eager", action="store_true", help="launch the rows one by one instead of replaying a graph")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with one Relu over 64 Mi floats (256 MiB read, 256 MiB written): the known-size "
                         "dispatch that scales FETCH_SIZE/WRITE_SIZE counters of a --pmc run")
    args = ap.parse_args(argv)
    device.init()
    if args.workload == "transfer":
        _transfer(max(args.runs, 1))
        return 0
    if args.workload == "rows":
        _rows(max(args.runs, 1))
        return 0
    g, inputs = BUILDERS[args.workload]()
    prog = Program(g)
    for name in g.inputs:
        prog.set_input(name, inputs[name])
    step = prog.run
    if not args.eager:
        prog.capture()
        step = prog.replay
    step()
    device.synchronize()
    start, stop = Event(), Event()
    start.record()
    for _ in range(args.runs):
        step()
    stop.record()
    ms = start.elapsed_ms(stop) / max(args.runs, 1)
    device.synchronize()
    prog.check_errors()
    print(f"{args.workload}: {ms:.3f} ms per {'eager run' if args.eager else 'replay'}, "
          f"{g.flops() / 1e9:.2f} GFLOP", flush=True)
    prog.close()
    if args.copy_probe:
        _copy_probe()
    return 0


def _copy_probe() -> None:
    """One Relu over 64 Mi non-negative floats: 256 MiB read, 256 MiB written."""
    import numpy as np

    from .device import DeviceArray, check, lib

    n = 64 << 20
    buf = DeviceArray.from_host(np.ones(n, np.float32))
    out = DeviceArray((n,), np.float32)
    check(lib().nert_hip_unary(0, 0, buf.ptr, out.ptr, n, 0.0, 0.0, None), "relu")
    device.synchronize()
    buf.close()
    out.close()


if __name__ == "__main__":
    sys.exit(main())
