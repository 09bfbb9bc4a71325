"""CPU: the on-disk model format -- nert_amd.graph's ONNX writer and reader.

The reference loader (src/model_loader.cpp, built into oracle/_ref) is the
oracle: every file the writer produces, with initializers embedded or in an
external-data side file, must load there and run to the same outputs, and the
reader must decode the same bytes to the values the reference executor sees
(each hand-encoded initializer is pushed through an Add node on the reference
and compared with `x + W` from our reader). External-data error cases must be
rejected by both, with the reference's message classes
(src/model_loader.cpp:326-365)."""

import os
import struct

import numpy as np
import pytest

from nert_amd import graph, workloads
from nert_amd.graph import _bytes, _int, _str, _value_info
from oracle import ref

BUILDERS = [
    ("resnet18", workloads.resnet18, {"batch": 1}),
    ("vit", workloads.vit_b16, {"batch": 1, "layers": 1}),
    ("detector", workloads.detector, {"batch": 1, "size": 128, "k": 50}),
]


def _same_graph(g, h):
    assert [n.op for n in h.nodes] == [n.op for n in g.nodes]
    assert h.inputs == g.inputs and h.outputs == g.outputs
    for a, b in zip(g.nodes, h.nodes):
        assert (a.inputs, a.outputs, a.name) == (b.inputs, b.outputs, b.name)
        assert set(a.attrs) == set(b.attrs), a.name
        for k, v in a.attrs.items():
            w = b.attrs[k]
            if isinstance(v, np.ndarray):
                assert v.dtype == w.dtype and np.array_equal(v, w), (a.name, k)
            elif isinstance(v, float):
                assert np.float32(v) == np.float32(w), (a.name, k)
            elif isinstance(v, (list, tuple)):
                assert [np.float32(x) if isinstance(x, float) else x for x in v] == \
                       [np.float32(x) if isinstance(x, float) else x for x in w], (a.name, k)
            else:
                assert int(v) == w if isinstance(v, (bool, np.bool_)) else v == w, (a.name, k)
    assert list(h.initializers) == list(g.initializers)
    for k, v in g.initializers.items():
        assert h.initializers[k].dtype == v.dtype and np.array_equal(h.initializers[k], v), k
    for k, (dt, shp) in g.tensors.items():
        assert (np.dtype(h.tensors[k][0]), tuple(h.tensors[k][1])) == (np.dtype(dt), tuple(shp)), k


@pytest.mark.parametrize("name,builder,kwargs", BUILDERS, ids=[b[0] for b in BUILDERS])
def test_round_trip_with_external_data(name, builder, kwargs, tmp_path):
    g, _ = builder(**kwargs)
    path = str(tmp_path / "model.onnx")
    files = graph.save_onnx(g, path, external_threshold=1024)
    assert len(files) == 2 and os.path.basename(files[1]) == "model.onnx.data"
    big = sum(v.nbytes for v in g.initializers.values() if v.nbytes >= 1024)
    side = os.path.getsize(files[1])
    assert big <= side < big + 64 * len(g.initializers)
    assert os.path.getsize(path) < 64 * 1024 + sum(v.nbytes for v in g.initializers.values() if v.nbytes < 1024)
    _same_graph(g, graph.load_onnx(path))
    # embedded form reads back the same
    path2 = str(tmp_path / "embedded.onnx")
    assert graph.save_onnx(g, path2) == [path2]
    _same_graph(g, graph.load_onnx(path2))


def _ref_outputs(path, g, inputs):
    lg = ref.LoadedGraph(path)
    try:
        outs = [np.zeros(g.tensors[t][1], g.tensors[t][0]) for t in g.outputs]
        ref.model_run(lg.handle, [inputs[n] for n in g.inputs], outs)
    finally:
        lg.close()
    return outs


@pytest.mark.parametrize("name,builder,kwargs", BUILDERS, ids=[b[0] for b in BUILDERS])
def test_reference_runs_external_file_identically(name, builder, kwargs, tmp_path):
    """The reference loader resolves the side file; its executor's outputs
    equal those of the embedded-weights file bit for bit, and equal those of
    the graph our reader returned, re-encoded."""
    g, inputs = builder(**kwargs)
    ext = str(tmp_path / "ext.onnx")
    emb = str(tmp_path / "emb.onnx")
    graph.save_onnx(g, ext, external_threshold=256)
    graph.save_onnx(g, emb)
    again = str(tmp_path / "again.onnx")
    graph.save_onnx(graph.load_onnx(ext), again, external_threshold=4096)
    want = _ref_outputs(emb, g, inputs)
    for p in (ext, again):
        for a, b in zip(_ref_outputs(p, g, inputs), want):
            assert a.dtype == b.dtype and np.array_equal(a, b), p


# ------------------------------------------------------ hand-encoded models ---

def _model(nodes, inits, inputs, outputs, value_info=()):
    body = b"".join(_bytes(1, n) for n in nodes) + _str(2, "t")
    body += b"".join(_bytes(5, t) for t in inits)
    body += b"".join(_bytes(11, _value_info(*i)) for i in inputs)
    body += b"".join(_bytes(12, _value_info(*o)) for o in outputs)
    body += b"".join(_bytes(13, _value_info(*v)) for v in value_info)
    return _int(1, 8) + _bytes(7, body) + _bytes(8, _str(1, "") + _int(2, 17))


def _node(op, ins, outs, name, attrs=b""):
    return b"".join(_str(1, i) for i in ins) + b"".join(_str(2, o) for o in outs) + _str(3, name) + \
        _str(4, op) + attrs


def _tensor_head(name, dtype, dims):
    return b"".join(_int(1, d) for d in dims) + _int(2, dtype) + _str(8, name)


def _ext(location=None, offset=None, length=None):
    out = b""
    for k, v in (("location", location), ("offset", offset), ("length", length)):
        if v is not None:
            out += _bytes(13, _str(1, k) + _str(2, str(v)))
    return out + _int(14, 1)


def _write(tmp_path, data, name="m.onnx"):
    p = str(tmp_path / name)
    with open(p, "wb") as f:
        f.write(data)
    return p


def _add_model(w_tensor, dtype, shape):
    np_dt = np.float32 if dtype == np.float32 else np.int64
    return _model([_node("Add", ["x", "W"], ["y"], "add")], [w_tensor], [("x", np_dt, shape)],
                  [("y", np_dt, shape)])


def _check_add(tmp_path, w_tensor, np_dt, shape, want_w, seed=0):
    """Reference Add(x, W) on the encoded W must equal x + our decoded W, and
    our decoded W must equal `want_w`."""
    p = _write(tmp_path, _add_model(w_tensor, np_dt, shape))
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape).astype(np.float32) if np_dt == np.float32
         else rng.integers(-1000, 1000, shape, dtype=np.int64))
    lg = ref.LoadedGraph(p)
    y = np.zeros(shape, np_dt)
    try:
        ref.model_run(lg.handle, [x], [y])
    finally:
        lg.close()
    h = graph.load_onnx(p)
    w = h.initializers["W"]
    assert w.dtype == np.dtype(np_dt) and w.shape == tuple(shape)
    assert np.array_equal(w, want_w)
    assert np.array_equal(y, x + w)


def test_typed_float_fields(tmp_path):
    w = np.random.default_rng(1).standard_normal((3, 5)).astype(np.float32)
    packed = _tensor_head("W", 1, w.shape) + _bytes(4, w.astype("<f4").tobytes())
    _check_add(tmp_path, packed, np.float32, w.shape, w)
    unpacked = _tensor_head("W", 1, w.shape) + b"".join(graph._key(4, 5) + struct.pack("<f", v)
                                                       for v in w.ravel())
    _check_add(tmp_path, unpacked, np.float32, w.shape, w)


def test_double_initializer_narrowed(tmp_path):
    d = np.random.default_rng(2).standard_normal((4, 6))
    raw = _tensor_head("W", 11, d.shape) + _bytes(9, d.astype("<f8").tobytes())
    _check_add(tmp_path, raw, np.float32, d.shape, d.astype(np.float32))
    typed = _tensor_head("W", 11, d.shape) + _bytes(10, d.astype("<f8").tobytes())
    _check_add(tmp_path, typed, np.float32, d.shape, d.astype(np.float32))


def test_integer_initializer_fields(tmp_path):
    v = np.array([[-5, 0, 7], [1 << 40, -(1 << 35), 3]], np.int64)
    packed = _tensor_head("W", 7, v.shape) + _bytes(7, b"".join(graph._varint(int(x)) for x in v.ravel()))
    _check_add(tmp_path, packed, np.int64, v.shape, v)
    unpacked = _tensor_head("W", 7, v.shape) + b"".join(_int(7, int(x)) for x in v.ravel())
    _check_add(tmp_path, unpacked, np.int64, v.shape, v)
    v32 = np.array([[-5, 0, 7], [70000, -3, 2]], np.int64)
    raw32 = _tensor_head("W", 6, v32.shape) + _bytes(9, v32.astype("<i4").tobytes())
    _check_add(tmp_path, raw32, np.int64, v32.shape, v32)
    typed32 = _tensor_head("W", 6, v32.shape) + _bytes(5, b"".join(graph._varint(int(x)) for x in v32.ravel()))
    _check_add(tmp_path, typed32, np.int64, v32.shape, v32)


def test_external_offset_absolute_location_and_open_length(tmp_path):
    w = np.arange(12, dtype=np.float32).reshape(3, 4) * 0.25 - 1
    side = tmp_path / "weights.bin"
    side.write_bytes(b"\x7f" * 100 + w.tobytes())
    # relative location, explicit offset and length
    rel = _tensor_head("W", 1, w.shape) + _ext("weights.bin", 100, w.nbytes)
    _check_add(tmp_path, rel, np.float32, w.shape, w)
    # absolute location, no length: read to the end of the file
    absolute = _tensor_head("W", 1, w.shape) + _ext(str(side), 100)
    _check_add(tmp_path, absolute, np.float32, w.shape, w)


@pytest.mark.parametrize("case,message", [
    ("missing_file", "cannot open external tensor data"),
    ("truncated", "truncated external tensor data"),
    ("no_location", "missing external data location"),
    ("wrong_count", "does not match shape"),
])
def test_external_errors_match_reference(case, message, tmp_path):
    w = np.ones((2, 3), np.float32)
    (tmp_path / "w.bin").write_bytes(w.tobytes())
    tensor = _tensor_head("W", 1, w.shape) + {
        "missing_file": _ext("absent.bin", 0, w.nbytes),
        "truncated": _ext("w.bin", 8, w.nbytes),
        "no_location": _ext(None, 0, w.nbytes),
        "wrong_count": _ext("w.bin", 4),
    }[case]
    p = _write(tmp_path, _add_model(tensor, np.float32, w.shape))
    with pytest.raises(ref.RefError, match=message):
        ref.LoadedGraph(p)
    with pytest.raises(graph.OnnxLoadError, match=message):
        graph.load_onnx(p)


def test_constant_nodes_and_repeated_initializer_inputs(tmp_path):
    """Constant nodes become initializers; a graph input naming an
    initializer stays a runtime input, as in the reference loader (which
    then expects it to be fed)."""
    c = np.array([1.5, -2.0, 3.25], np.float32)
    attr = _bytes(5, _str(1, "value") + _bytes(5, _tensor_head("", 1, c.shape) + _bytes(9, c.tobytes())) +
                  _int(20, 4))
    b = np.array([0.5, 0.5, 0.5], np.float32)
    nodes = [_node("Constant", [], ["c"], "const", attr), _node("Add", ["x", "c"], ["t"], "add"),
             _node("Mul", ["t", "B"], ["y"], "mul")]
    data = _model(nodes, [_tensor_head("B", 1, b.shape) + _bytes(9, b.tobytes())],
                  [("x", np.float32, (3,)), ("B", np.float32, (3,))], [("y", np.float32, (3,))],
                  [("t", np.float32, (3,))])
    p = _write(tmp_path, data)
    h = graph.load_onnx(p)
    assert [n.op for n in h.nodes] == ["Add", "Mul"]
    assert h.inputs == ["x", "B"] and h.outputs == ["y"]
    assert np.array_equal(h.initializers["c"], c) and np.array_equal(h.initializers["B"], b)
    x = np.array([1.0, 2.0, 3.0], np.float32)
    y = np.zeros(3, np.float32)
    lg = ref.LoadedGraph(p)
    try:
        ref.model_run(lg.handle, [x, b], [y])
    finally:
        lg.close()
    assert np.array_equal(y, (x + c) * b)


def test_reader_needs_intermediate_shapes(tmp_path):
    g, _ = workloads.detector(batch=1, size=64, k=10)
    p = _write(tmp_path, graph.to_onnx(g))  # no value_info for intermediates
    with pytest.raises(graph.OnnxLoadError, match="no dtype/shape recorded"):
        graph.load_onnx(p)
