"""Replays one of the seeded BASELINE workloads through the runner, for
timing and kernel traces:

    python3 -m nert_amd.replay {resnet18,vit,detector} [--runs N]

Builds the program (Conv chain fusion, view aliasing), binds the seeded
input, runs it once eagerly (per-geometry kernel choices are made here),
captures it into a HIP graph and replays it N times between HIP events on
the layer stream. Prints one line: workload, ms per replay, and the
algorithmic GFLOP of the graph.
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


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("workload", choices=sorted(BUILDERS))
    ap.add_argument("--runs", type=int, default=10)
    args = ap.parse_args(argv)
    device.init()
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
