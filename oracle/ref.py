"""ctypes loader for the reference CPU oracle (oracle/_ref/libnert_refshim.so).

Test infrastructure only: see oracle/__init__.py.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from nert_amd import abi

REF_DIR = Path(__file__).resolve().parent / "_ref"
SHIM = REF_DIR / "libnert_refshim.so"


class RefError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.message = message


_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not SHIM.exists():
            raise RuntimeError(f"{SHIM} is not built; run `make -C oracle`")
        L = C.CDLL(str(SHIM), mode=C.RTLD_GLOBAL)
        L.nert_ref_run_node.argtypes = abi.node_argtypes()
        L.nert_ref_has_row.argtypes = [C.c_char_p]
        L.nert_ref_model_run.argtypes = [C.c_void_p, C.c_int, C.POINTER(abi.TensorDesc), C.c_int,
                                         C.POINTER(abi.TensorDesc), C.POINTER(C.c_double), C.c_char_p, C.c_int]
        L.nert_ref_infer_shape.argtypes = [C.c_void_p, C.c_int, C.POINTER(abi.TensorDesc), C.c_char_p,
                                           C.POINTER(C.c_int64), C.POINTER(C.c_int), C.c_char_p, C.c_int]
        L.nert_ref_load_graph.restype = C.c_void_p
        L.nert_ref_load_graph.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
        L.nert_ref_free_graph.argtypes = [C.c_void_p]
        _lib = L
    return _lib


class LoadedGraph:
    """A nert::Graph loaded from an ONNX file by the reference loader."""

    def __init__(self, path: str):
        err = C.create_string_buffer(4096)
        self.handle = lib().nert_ref_load_graph(str(path).encode(), err, len(err))
        if not self.handle:
            raise RefError(abi.OTHER_ERROR, err.value.decode())

    def close(self) -> None:
        if self.handle:
            lib().nert_ref_free_graph(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def has_row(op_type: str) -> bool:
    return bool(lib().nert_ref_has_row(op_type.encode()))


def run_node(op_type: str, inputs: Sequence[np.ndarray | None], outputs: Sequence[np.ndarray],
             attrs: dict[str, Any] | None = None, name: str = "n", schema_version: int = 0) -> None:
    """Runs one CpuDevice row on host arrays, writing `outputs` in place."""
    ap = abi.AttrPack(attrs)
    ip = abi.TensorPack(abi.host_entries(inputs))
    op = abi.TensorPack(abi.host_entries(outputs))
    err = C.create_string_buffer(4096)
    rc = lib().nert_ref_run_node(op_type.encode(), name.encode(), schema_version, ap.array, ap.count, ip.array,
                                 ip.count, op.array, op.count, err, len(err))
    if rc != abi.OK:
        raise RefError(rc, err.value.decode())


def model_run(graph_handle: int, inputs: Sequence[np.ndarray], outputs: Sequence[np.ndarray]) -> float:
    """Runs a nert::Graph through Model(graph, dims, CpuDevice()).RunTyped;
    returns the seconds RunTyped took."""
    ip = abi.TensorPack(abi.host_entries(inputs))
    op = abi.TensorPack(abi.host_entries(outputs))
    secs = C.c_double()
    err = C.create_string_buffer(4096)
    rc = lib().nert_ref_model_run(graph_handle, ip.count, ip.array, op.count, op.array, C.byref(secs), err, len(err))
    if rc != abi.OK:
        raise RefError(rc, err.value.decode())
    return float(secs.value)


def infer_shape(graph_handle: int, inputs: Sequence[np.ndarray], name: str) -> tuple[int, ...]:
    ip = abi.TensorPack(abi.host_entries(inputs))
    dims = (C.c_int64 * 8)()
    rank = C.c_int()
    err = C.create_string_buffer(4096)
    rc = lib().nert_ref_infer_shape(graph_handle, ip.count, ip.array, name.encode(), dims, C.byref(rank), err,
                                    len(err))
    if rc != abi.OK:
        raise RefError(rc, err.value.decode())
    return tuple(int(dims[i]) for i in range(rank.value))
