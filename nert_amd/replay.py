"""Replays one of the seeded BASELINE workloads through the runner, for
timing and kernel traces:

    python3 -m nert_amd.replay {resnet18,vit,detector} [--runs N]

Builds the program (Conv chain fusion, view aliasing), binds the seeded
input, runs it once eagerly (per-geometry kernel choices are made here),
captures it into a HIP graph and replays it N times between HIP events on
the layer stream. Prints one line: workload, ms per replay, and the
algorithmic GFLOP of the graph.

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


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("workload", choices=sorted(BUILDERS) + ["transfer"])
    ap.add_argument("--runs", type=int, default=10)
    args = ap.parse_args(argv)
    device.init()
    if args.workload == "transfer":
        _transfer(max(args.runs, 1))
        return 0
    g, inputs = BUILDERS[args.workload]()
    prog = Program(g)
    for name in g.inputs:
        prog.set_input(name, inputs[name])
    prog.capture()
    prog.replay()
    device.synchronize()
    start, stop = Event(), Event()
    start.record()
    for _ in range(args.runs):
        prog.replay()
    stop.record()
    ms = start.elapsed_ms(stop) / max(args.runs, 1)
    device.synchronize()
    print(f"{args.workload}: {ms:.3f} ms per replay, {g.flops() / 1e9:.2f} GFLOP", flush=True)
    prog.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
