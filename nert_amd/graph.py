"""A minimal graph description for synthetic workloads, and its ONNX encoding.

A `Graph` holds nodes in execution order, named initializers (numpy arrays),
declared inputs/outputs and the dtype/shape of every tensor -- the same
information nert::Graph carries (include/nert/graph.hpp:178-239). `to_onnx()`
writes it as an ONNX ModelProto (opset 17) with a hand-rolled protobuf encoder,
so the reference's own loader (src/model_loader.cpp:2278 LoadGraphFromFile)
reads the very model the gfx950 runner executes. The `onnx` package is not
needed (the reference's tests encode models the same way,
test/loader_test.cpp:49-340).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Any

import numpy as np

# ONNX TensorProto.DataType codes
ONNX_FLOAT, ONNX_INT64, ONNX_BOOL = 1, 7, 9
_NP_TO_ONNX = {np.dtype(np.float32): ONNX_FLOAT, np.dtype(np.int64): ONNX_INT64, np.dtype(np.bool_): ONNX_BOOL}


@dataclass
class Node:
    op: str
    inputs: list[str]
    outputs: list[str]
    attrs: dict[str, Any] = field(default_factory=dict)
    name: str = ""


@dataclass
class Graph:
    nodes: list[Node] = field(default_factory=list)
    initializers: dict[str, np.ndarray] = field(default_factory=dict)
    inputs: list[str] = field(default_factory=list)
    outputs: list[str] = field(default_factory=list)
    # name -> (numpy dtype, shape) for every tensor
    tensors: dict[str, tuple[np.dtype, tuple[int, ...]]] = field(default_factory=dict)

    def add_initializer(self, name: str, value: np.ndarray) -> str:
        self.initializers[name] = value
        self.tensors[name] = (value.dtype, tuple(value.shape))
        return name

    def add_input(self, name: str, dtype: Any, shape: tuple[int, ...]) -> str:
        self.inputs.append(name)
        self.tensors[name] = (np.dtype(dtype), tuple(shape))
        return name

    def add_node(self, op: str, inputs: list[str], output_specs: list[tuple[str, Any, tuple[int, ...]]],
                 attrs: dict[str, Any] | None = None, name: str | None = None) -> list[str]:
        outs = []
        for oname, dtype, shape in output_specs:
            self.tensors[oname] = (np.dtype(dtype), tuple(int(s) for s in shape))
            outs.append(oname)
        self.nodes.append(Node(op, list(inputs), outs, dict(attrs or {}), name or f"{op.lower()}_{len(self.nodes)}"))
        return outs

    def flops(self, op: str | None = None) -> int:
        """Algorithmic multiply-add flops (2 per MAC) of Conv/Gemm/MatMul nodes."""
        total = 0
        for n in self.nodes:
            if op is not None and n.op != op:
                continue
            if n.op == "Conv":
                w = self.tensors[n.inputs[1]][1]
                y = self.tensors[n.outputs[0]][1]
                total += 2 * int(np.prod(y)) * int(np.prod(w[1:]))
            elif n.op in ("Gemm", "MatMul"):
                a = self.tensors[n.inputs[0]][1]
                y = self.tensors[n.outputs[0]][1]
                if n.op == "Gemm":
                    k = a[0] if n.attrs.get("transA", 0) else a[1]
                else:
                    k = a[-1]
                total += 2 * int(np.prod(y)) * int(k)
        return total


# ---------------------------------------------------------------- protobuf ---

def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field_no: int, wire: int) -> bytes:
    return _varint((field_no << 3) | wire)


def _int(field_no: int, v: int) -> bytes:
    return _key(field_no, 0) + _varint(int(v))


def _bytes(field_no: int, b: bytes) -> bytes:
    return _key(field_no, 2) + _varint(len(b)) + b


def _str(field_no: int, s: str) -> bytes:
    return _bytes(field_no, s.encode())


def _float(field_no: int, f: float) -> bytes:
    return _key(field_no, 5) + struct.pack("<f", f)


class ExternalData:
    """Collects initializer payloads that go to a side file instead of the
    model's raw_data fields. Each payload starts on an `align`-byte boundary of
    the side file; `location` is written as given (relative paths resolve
    against the model file's directory, src/model_loader.cpp:337-340)."""

    def __init__(self, location: str, threshold: int = 1024, align: int = 64):
        self.location = location
        self.threshold = int(threshold)
        self.align = int(align)
        self.blob = bytearray()

    def place(self, raw: bytes) -> tuple[int, int]:
        offset = -len(self.blob) % self.align + len(self.blob)
        self.blob.extend(b"\0" * (offset - len(self.blob)))
        self.blob.extend(raw)
        return offset, len(raw)


def _tensor(name: str, a: np.ndarray, external: ExternalData | None = None) -> bytes:
    out = b"".join(_int(1, d) for d in a.shape)
    out += _int(2, _NP_TO_ONNX[a.dtype])
    out += _str(8, name)
    raw = np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
    if external is not None and len(raw) >= external.threshold:
        offset, length = external.place(raw)
        for key, value in (("location", external.location), ("offset", str(offset)), ("length", str(length))):
            out += _bytes(13, _str(1, key) + _str(2, value))
        out += _int(14, 1)
        return out
    out += _bytes(9, raw)
    return out


def _attribute(name: str, value: Any) -> bytes:
    out = _str(1, name)
    if isinstance(value, (bool, np.bool_)):
        return out + _int(3, int(value)) + _int(20, 2)
    if isinstance(value, (float, np.floating)):
        return out + _float(2, float(value)) + _int(20, 1)
    if isinstance(value, (int, np.integer)):
        return out + _int(3, int(value)) + _int(20, 2)
    if isinstance(value, str):
        return out + _bytes(4, value.encode()) + _int(20, 3)
    if isinstance(value, np.ndarray):
        return out + _bytes(5, _tensor("", value)) + _int(20, 4)
    if isinstance(value, (list, tuple)):
        if value and all(isinstance(v, (float, np.floating)) for v in value):
            return out + _bytes(7, b"".join(struct.pack("<f", v) for v in value)) + _int(20, 6)
        return out + _bytes(8, b"".join(_varint(int(v)) for v in value)) + _int(20, 7)
    raise TypeError(f"attribute {name}: unsupported value {value!r}")


def _value_info(name: str, dtype: np.dtype, shape: tuple[int, ...]) -> bytes:
    dims = b"".join(_bytes(1, _int(1, d)) for d in shape)
    tensor_type = _int(1, _NP_TO_ONNX[np.dtype(dtype)]) + _bytes(2, dims)
    return _str(1, name) + _bytes(2, _bytes(1, tensor_type))


def to_onnx(g: Graph, opset: int = 17, graph_name: str = "synthetic", value_info: bool = False,
            external: ExternalData | None = None) -> bytes:
    """Serialises `g` as an ONNX ModelProto (ir_version 8, ai.onnx opset `opset`).

    value_info=True also records the dtype/shape of every intermediate tensor
    (GraphProto.value_info, read by src/model_loader.cpp:2165-2186), which makes
    the file self-describing for `from_onnx`. With `external`, initializers of
    at least `external.threshold` bytes are stored in `external.blob` and
    referenced by location/offset/length with data_location EXTERNAL
    (src/model_loader.cpp:287-317); the caller writes the blob to that location.
    """
    body = b""
    for n in g.nodes:
        nb = b"".join(_str(1, i) for i in n.inputs) + b"".join(_str(2, o) for o in n.outputs)
        nb += _str(3, n.name) + _str(4, n.op)
        nb += b"".join(_bytes(5, _attribute(k, v)) for k, v in n.attrs.items())
        body += _bytes(1, nb)
    body += _str(2, graph_name)
    for name, a in g.initializers.items():
        body += _bytes(5, _tensor(name, a, external))
    for name in g.inputs:
        dt, shp = g.tensors[name]
        body += _bytes(11, _value_info(name, dt, shp))
    for name in g.outputs:
        dt, shp = g.tensors[name]
        body += _bytes(12, _value_info(name, dt, shp))
    if value_info:
        declared = set(g.inputs) | set(g.outputs) | set(g.initializers)
        for n in g.nodes:
            for o in n.outputs:
                if o and o not in declared and o in g.tensors:
                    dt, shp = g.tensors[o]
                    body += _bytes(13, _value_info(o, dt, shp))
                    declared.add(o)
    model = _int(1, 8) + _str(2, "nert_amd") + _bytes(7, body) + _bytes(8, _str(1, "") + _int(2, opset))
    return model


def save_onnx(g: Graph, path: str, external_threshold: int | None = None, value_info: bool = True,
              opset: int = 17) -> list[str]:
    """Writes `g` to `path`; with `external_threshold` set, initializers of at
    least that many bytes go to `<path>.data` beside it (location stored
    relative to the model's directory). Returns the files written."""
    import os
    ext = None
    if external_threshold is not None:
        ext = ExternalData(os.path.basename(path) + ".data", threshold=external_threshold)
    data = to_onnx(g, opset=opset, value_info=value_info, external=ext)
    with open(path, "wb") as f:
        f.write(data)
    written = [path]
    if ext is not None:
        side = os.path.join(os.path.dirname(os.path.abspath(path)), ext.location)
        with open(side, "wb") as f:
            f.write(bytes(ext.blob))
        written.append(side)
    return written


# ------------------------------------------------------------------ reader ---

class OnnxLoadError(ValueError):
    """A model file the reader cannot turn into a Graph; the messages follow
    the reference loader's (src/model_loader.cpp:326-365)."""


_ONNX_TO_NP = {1: np.dtype(np.float32), 11: np.dtype(np.float32), 7: np.dtype(np.int64), 6: np.dtype(np.int64),
               9: np.dtype(np.bool_)}


def _fields(buf: bytes):
    """Yields (field_no, wire_type, value) over one protobuf message; value is
    an int for varint/fixed fields and a memoryview for length-delimited ones."""
    mv = memoryview(buf)
    i, n = 0, len(mv)

    def varint():
        nonlocal i
        shift = value = 0
        while True:
            if i >= n:
                raise OnnxLoadError("truncated varint")
            b = mv[i]
            i += 1
            value |= (b & 0x7F) << shift
            if b < 0x80:
                return value
            shift += 7

    while i < n:
        key = varint()
        fno, wire = key >> 3, key & 7
        if wire == 0:
            yield fno, wire, varint()
        elif wire == 1:
            if i + 8 > n:
                raise OnnxLoadError("truncated fixed64")
            yield fno, wire, int.from_bytes(mv[i:i + 8], "little")
            i += 8
        elif wire == 2:
            ln = varint()
            if i + ln > n:
                raise OnnxLoadError("truncated length-delimited field")
            yield fno, wire, mv[i:i + ln]
            i += ln
        elif wire == 5:
            if i + 4 > n:
                raise OnnxLoadError("truncated fixed32")
            yield fno, wire, int.from_bytes(mv[i:i + 4], "little")
            i += 4
        else:
            raise OnnxLoadError(f"unsupported wire type {wire}")


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _packed_varints(wire: int, value) -> list[int]:
    """Repeated int64 field: one varint (wire 0) or a packed run (wire 2)."""
    if wire == 0:
        return [_signed(value)]
    out, shift, acc = [], 0, 0
    for b in bytes(value):
        acc |= (b & 0x7F) << shift
        if b < 0x80:
            out.append(_signed(acc))
            shift = acc = 0
        else:
            shift += 7
    if shift:
        raise OnnxLoadError("truncated packed varint")
    return out


def _packed_f32(wire: int, value) -> list[float]:
    if wire == 5:
        return [struct.unpack("<f", value.to_bytes(4, "little"))[0]]
    return list(np.frombuffer(bytes(value), dtype="<f4").astype(np.float32))


def _packed_f64(wire: int, value) -> list[float]:
    if wire == 1:
        return [struct.unpack("<d", value.to_bytes(8, "little"))[0]]
    return list(np.frombuffer(bytes(value), dtype="<f8"))


def _read_external(name: str, location: str, offset: int, length: int, model_dir: str) -> bytes:
    """Payload of an EXTERNAL tensor (src/model_loader.cpp:326-365): a
    relative location resolves against the model's directory, a missing
    length means "to the end of the file", a short read is an error."""
    import os
    if not location:
        raise OnnxLoadError(f"missing external data location for tensor '{name}'")
    full = location if location.startswith("/") else os.path.join(model_dir, location)
    try:
        f = open(full, "rb")
    except OSError:
        raise OnnxLoadError(f"cannot open external tensor data for tensor '{name}' at {full}") from None
    with f:
        f.seek(offset)
        data = f.read() if length < 0 else f.read(length)
    if length >= 0 and len(data) != length:
        raise OnnxLoadError(f"truncated external tensor data for tensor '{name}' at {full}")
    return data


def _decode_tensor(buf, model_dir: str) -> tuple[str, np.ndarray]:
    dims: list[int] = []
    dtype = 0
    name = ""
    raw = None
    floats: list[float] = []
    ints: list[int] = []
    int32s: list[int] = []
    doubles: list[float] = []
    ext: dict[str, str] = {}
    external = False
    for fno, wire, v in _fields(buf):
        if fno == 1:
            dims += _packed_varints(wire, v)
        elif fno == 2:
            dtype = v
        elif fno == 4:
            floats += _packed_f32(wire, v)
        elif fno == 5:
            int32s += _packed_varints(wire, v)
        elif fno == 7:
            ints += _packed_varints(wire, v)
        elif fno == 8:
            name = bytes(v).decode()
        elif fno == 9:
            raw = bytes(v)
        elif fno == 10:
            doubles += _packed_f64(wire, v)
        elif fno == 13:
            entry = {k: bytes(x).decode() for k, _, x in _fields(v) if k in (1, 2)}
            ext[entry.get(1, "")] = entry.get(2, "")
        elif fno == 14:
            external = v == 1
    if dtype not in _ONNX_TO_NP:
        raise OnnxLoadError(f"unsupported initializer data type {dtype} for tensor '{name}'")
    count = int(np.prod(dims)) if dims else 1

    def payload() -> bytes:
        if external:
            return _read_external(name, ext.get("location", ""), int(ext.get("offset", "0")),
                                  int(ext.get("length", "-1")), model_dir)
        return raw or b""

    if dtype == 1:
        values = np.asarray(floats, np.float32) if floats else np.frombuffer(payload(), "<f4")
    elif dtype == 11:
        values = np.asarray(doubles, np.float64) if doubles else np.frombuffer(payload(), "<f8")
    elif dtype == 7:
        values = np.asarray(ints, np.int64) if ints else np.frombuffer(payload(), "<i8")
    elif dtype == 6:
        values = np.asarray(int32s, np.int64) if int32s else np.frombuffer(payload(), "<i4")
    else:
        values = np.asarray(int32s, np.int64) if int32s else np.frombuffer(payload(), np.uint8)
    if values.size != count:
        raise OnnxLoadError(f"initializer element count {values.size} does not match shape for tensor '{name}'")
    return name, values.astype(_ONNX_TO_NP[dtype]).reshape(dims)


def _decode_attribute(buf, model_dir: str) -> tuple[str, Any]:
    name, kind = "", 0
    f = i = s = t = None
    fl: list[float] = []
    il: list[int] = []
    sl: list[str] = []
    for fno, wire, v in _fields(buf):
        if fno == 1:
            name = bytes(v).decode()
        elif fno == 2:
            f = struct.unpack("<f", v.to_bytes(4, "little"))[0]
        elif fno == 3:
            i = _signed(v)
        elif fno == 4:
            s = bytes(v).decode()
        elif fno == 5:
            t = _decode_tensor(v, model_dir)[1]
        elif fno == 7:
            fl += _packed_f32(wire, v)
        elif fno == 8:
            il += _packed_varints(wire, v)
        elif fno == 9:
            sl.append(bytes(v).decode())
        elif fno == 20:
            kind = v
    by_kind = {1: f, 2: i, 3: s, 4: t, 6: [float(x) for x in fl], 7: il, 8: sl}
    if kind in by_kind:
        value = by_kind[kind]
        if value is None:
            raise OnnxLoadError(f"attribute '{name}' declares type {kind} but carries no value")
        return name, value
    for value in (f, i, s, t):
        if value is not None:
            return name, value
    return name, [float(x) for x in fl] if fl else (il if il else sl)


def _decode_value_info(buf) -> tuple[str, np.dtype, tuple[int, ...]]:
    name, elem, dims = "", 0, []
    for fno, _, v in _fields(buf):
        if fno == 1:
            name = bytes(v).decode()
        elif fno == 2:
            for tf, _, tt in _fields(v):
                if tf != 1:
                    continue
                for ff, _, fv in _fields(tt):
                    if ff == 1:
                        elem = fv
                    elif ff == 2:
                        for df, _, dim in _fields(fv):
                            if df != 1:
                                continue
                            value = None
                            for kf, _, kv in _fields(dim):
                                if kf == 1:
                                    value = _signed(kv)
                            if value is None:
                                raise OnnxLoadError(f"tensor '{name}' has a symbolic dimension")
                            dims.append(value)
    if elem not in _ONNX_TO_NP:
        raise OnnxLoadError(f"unsupported element type {elem} for tensor '{name}'")
    return name, _ONNX_TO_NP[elem], tuple(dims)


def from_onnx(data: bytes, model_dir: str = ".") -> Graph:
    """Decodes an ONNX ModelProto into a Graph -- the reader half of the
    round trip with `to_onnx`, covering the subset nert's loader accepts
    (src/model_loader.cpp:2080-2200): raw_data, typed data fields and external
    data for initializers (DOUBLE narrowed to float32, INT32 widened to int64,
    as src/model_loader.cpp:376-392 does), Constant nodes folded into
    initializers. A graph input that repeats an initializer's name stays a
    graph input, as in src/model_loader.cpp:2141-2152. Every node output needs
    a dtype/shape entry (graph output or value_info)."""
    g = Graph()
    graph_buf = None
    for fno, _, v in _fields(data):
        if fno == 7:
            graph_buf = v
    if graph_buf is None:
        raise OnnxLoadError("model has no graph")
    declared_inputs: list[str] = []
    for fno, _, v in _fields(graph_buf):
        if fno == 1:
            node = Node("", [], [])
            for nf, _, nv in _fields(v):
                if nf == 1:
                    node.inputs.append(bytes(nv).decode())
                elif nf == 2:
                    node.outputs.append(bytes(nv).decode())
                elif nf == 3:
                    node.name = bytes(nv).decode()
                elif nf == 4:
                    node.op = bytes(nv).decode()
                elif nf == 5:
                    k, a = _decode_attribute(nv, model_dir)
                    node.attrs[k] = a
            if node.op == "Constant":
                value = node.attrs.get("value")
                if value is None:
                    for key, dt in (("value_float", np.float32), ("value_floats", np.float32),
                                    ("value_int", np.int64), ("value_ints", np.int64)):
                        if key in node.attrs:
                            value = np.asarray(node.attrs[key], dt)
                if value is None:
                    raise OnnxLoadError(f"Constant node '{node.name}' carries no supported value")
                g.add_initializer(node.outputs[0], np.asarray(value))
                continue
            g.nodes.append(node)
        elif fno == 5:
            name, value = _decode_tensor(v, model_dir)
            g.add_initializer(name, value)
        elif fno in (11, 12, 13):
            name, dt, shp = _decode_value_info(v)
            if fno == 11:
                declared_inputs.append(name)
            elif fno == 12:
                g.outputs.append(name)
            g.tensors.setdefault(name, (dt, shp))
    g.inputs = declared_inputs
    for n in g.nodes:
        for o in n.outputs:
            if o and o not in g.tensors:
                raise OnnxLoadError(f"no dtype/shape recorded for tensor '{o}' (write the model with value_info)")
    return g


def load_onnx(path: str) -> Graph:
    """Reads a model file written by `save_onnx` (or any model in the subset
    `from_onnx` covers); external data resolves against the file's directory."""
    import os
    with open(path, "rb") as f:
        data = f.read()
    return from_onnx(data, os.path.dirname(os.path.abspath(path)))
