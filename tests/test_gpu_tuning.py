"""Reproducibility across processes.

A tile shape or split-K count fixes the order in which a Conv/Gemm sum is
formed, so it fixes the rounding. The committed table
(nert_amd/tuning/gfx950.tsv) holds the choice for every geometry of the
seeded BASELINE workloads, so two fresh processes run them with the same
kernels and give the same bits. Each workload runs in a child process with
NERT_HIP_TUNE_LOG=1, which prints one line per table lookup and, for a
geometry the table lacks, one line per timed candidate.
"""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = """
import sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd import workloads
from nert_amd.runner import Program

g, inputs = workloads.{builder}(batch={batch})
prog = Program(g)
for n in g.inputs:
    prog.set_input(n, inputs[n])
prog.run()
prog.capture()
prog.replay()
np.savez({path!r}, **{{f"out{{i}}": prog.output(t) for i, t in enumerate(g.outputs)}})
prog.close()
print("child done", flush=True)
"""


def _child(builder: str, batch: int, path: str) -> tuple[dict[str, np.ndarray], str]:
    env = dict(os.environ, NERT_HIP_TUNE_LOG="1")
    env.pop("NERT_HIP_CONV_TUNE", None)
    env.pop("NERT_HIP_TUNE_TABLE", None)
    print(f"child: {builder} batch {batch}", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD.format(root=ROOT, builder=builder, batch=batch, path=path)],
                       env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, f"{builder} child exited {r.returncode}:\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}"
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}, r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("builder,batch", [("resnet18", 32), ("vit_b16", 16), ("detector", 8)])
def test_workload_bits_same_across_processes(gpu, tmp_path, builder, batch):
    """Two fresh processes, the same seeded model and input: every Conv and
    Gemm geometry comes from the committed table (no candidate is timed),
    and the outputs are bit-identical."""
    runs = [_child(builder, batch, str(tmp_path / f"run{i}.npz")) for i in range(2)]
    for _, log in runs:
        lines = [ln for ln in log.splitlines() if ln.startswith("nert_hip tune:")]
        timed = [ln for ln in lines if " chose " in ln]
        assert not timed, f"{builder}: geometries missing from the committed table:\n" + "\n".join(timed)
        assert any(" table " in ln for ln in lines), f"{builder}: no table lookups logged"
    (a, _), (b, _) = runs
    assert sorted(a) == sorted(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
        assert a[k].tobytes() == b[k].tobytes(), f"{builder} output {k} differs between processes"
