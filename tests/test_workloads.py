"""CPU: the seeded workloads (configs[2..4]) are valid ONNX for the reference.

For each builder, at a reduced size, the ONNX encoding loads in the
reference loader, the reference's shape inference agrees with the builder's
tensor table for every node output, and the reference executor runs it.
The GPU comparisons live in tests/test_gpu_workloads.py."""

import os
import tempfile

import numpy as np
import pytest

from nert_amd import graph, workloads
from oracle import ref


def _load(g):
    path = os.path.join(tempfile.mkdtemp(), "m.onnx")
    with open(path, "wb") as f:
        f.write(graph.to_onnx(g))
    return ref.LoadedGraph(path)


def _check_shapes(g, inputs):
    lg = _load(g)
    try:
        feeds = [inputs[n] for n in g.inputs]
        for n in g.nodes:
            for t in n.outputs:
                assert ref.infer_shape(lg.handle, feeds, t) == tuple(g.tensors[t][1]), (n.op, t)
    finally:
        lg.close()


@pytest.mark.parametrize("builder,kwargs", [
    (workloads.resnet18, {"batch": 1}),
    (workloads.vit_b16, {"batch": 1, "layers": 1}),
    (workloads.detector, {"batch": 1, "size": 128, "k": 50}),
])
def test_reference_infers_builder_shapes(builder, kwargs):
    g, inputs = builder(**kwargs)
    _check_shapes(g, inputs)


def test_detector_runs_on_reference():
    g, inputs = workloads.detector(batch=1, size=128, k=20)
    lg = _load(g)
    outs = [np.zeros(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
    ref.model_run(lg.handle, [inputs["input"]], outs)
    lg.close()
    scores, boxes, classes = outs
    assert np.all(np.diff(scores, axis=1) <= 0)          # sorted descending
    assert classes.dtype == np.int64 and classes.min() >= 0 and classes.max() < 80
    assert np.all(np.isfinite(boxes))


def test_vit_flops_match_config():
    g, _ = workloads.vit_b16(batch=16)
    assert abs(g.flops() / 1e9 - 562.04) < 0.01
