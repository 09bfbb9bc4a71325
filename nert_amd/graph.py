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


def _tensor(name: str, a: np.ndarray) -> bytes:
    out = b"".join(_int(1, d) for d in a.shape)
    out += _int(2, _NP_TO_ONNX[a.dtype])
    out += _str(8, name)
    raw = np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
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


def to_onnx(g: Graph, opset: int = 17, graph_name: str = "synthetic") -> bytes:
    """Serialises `g` as an ONNX ModelProto (ir_version 8, ai.onnx opset `opset`)."""
    body = b""
    for n in g.nodes:
        nb = b"".join(_str(1, i) for i in n.inputs) + b"".join(_str(2, o) for o in n.outputs)
        nb += _str(3, n.name) + _str(4, n.op)
        nb += b"".join(_bytes(5, _attribute(k, v)) for k, v in n.attrs.items())
        body += _bytes(1, nb)
    body += _str(2, graph_name)
    for name, a in g.initializers.items():
        body += _bytes(5, _tensor(name, a))
    for name in g.inputs:
        dt, shp = g.tensors[name]
        body += _bytes(11, _value_info(name, dt, shp))
    for name in g.outputs:
        dt, shp = g.tensors[name]
        body += _bytes(12, _value_info(name, dt, shp))
    model = _int(1, 8) + _str(2, "nert_amd") + _bytes(7, body) + _bytes(8, _str(1, "") + _int(2, opset))
    return model
