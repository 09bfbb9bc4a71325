"""Writes tests/golden/models/*.npz: the reference executor's outputs for the
seeded full-size workloads, so GPU tests can pin the deep stacks against the
oracle without a half-hour CPU run on the GPU box.

Each fixture holds the outputs of `nert::Model(graph, dims, CpuDevice())
.RunTyped` (olibartfast/nert src/executor.cpp:202-560, built in place by
oracle/Makefile into oracle/_ref) on the graph and input that
nert_amd.workloads builds for the config, plus fingerprints of that input and
of the weights (model_fixtures.fingerprint), so a test can tell a changed
generator from a wrong kernel.

    python tests/golden/make_model_fixtures.py [resnet18 vit detector]

Cases:
  resnet18_bs32  configs[2] at full size: logits [32,1000]           (~45 s)
  resnet18_bs1   configs[2]'s network at batch 1, the reference's own
                 full-model gate batch (tools/hip_model_check.cpp)   (~3 s)
  vit_bs2        configs[3] with all 12 layers at batch 2: logits [2,1000]
                 (the reference's naive MatMul makes batch 16 a half-hour
                 run; batch 2 exercises every layer)                 (~4 min)
  vit_bs16       configs[3] at full size: logits [16,1000], all 16 images
                                                                     (~30 min)
  detector_bs8   configs[4] at full size: top scores [8,300], boxes
                 [8,300,4], classes [8,300] int64                    (~20 s)
"""

from __future__ import annotations

import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from nert_amd import graph, workloads  # noqa: E402
from oracle import ref  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parent))
from model_fixtures import DIR as OUT, fingerprint  # noqa: E402

CASES = {
    "resnet18_bs32": lambda: workloads.resnet18(batch=32),
    "resnet18_bs1": lambda: workloads.resnet18(batch=1),
    "vit_bs2": lambda: workloads.vit_b16(batch=2, layers=12),
    "vit_bs16": lambda: workloads.vit_b16(batch=16, layers=12),
    "detector_bs8": lambda: workloads.detector(batch=8),
}


def run_reference(g, inputs: dict) -> tuple[list[np.ndarray], float]:
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.onnx")
        graph.save_onnx(g, path)
        lg = ref.LoadedGraph(path)
        outs = [np.zeros(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
        try:
            secs = ref.model_run(lg.handle, [inputs[n] for n in g.inputs], outs)
        finally:
            lg.close()
    return outs, secs


def make(name: str) -> Path:
    g, inputs = CASES[name]()
    t0 = time.time()
    outs, secs = run_reference(g, inputs)
    arrays = {f"out{i}_{t}": o for i, (t, o) in enumerate(zip(g.outputs, outs))}
    arrays["fingerprint"] = fingerprint(g, inputs)
    OUT.mkdir(parents=True, exist_ok=True)
    path = OUT / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    print(f"{name}: {', '.join(f'{k}{list(v.shape)}' for k, v in arrays.items())}; reference Run {secs:.1f} s "
          f"({time.time() - t0:.1f} s total) -> {path.relative_to(ROOT)}", flush=True)
    return path


if __name__ == "__main__":
    for case in sys.argv[1:] or list(CASES):
        make(case if case in CASES else {"resnet18": "resnet18_bs32", "vit": "vit_bs2",
                                          "detector": "detector_bs8"}[case])
