"""ctypes mirror of include/nert_abi.h: plain-C node and tensor descriptions.

No library is loaded here; both the device layer (nert_amd.device) and the test
oracle loader use these structures to describe a node the way the reference
seam does (nert::Node / nert::TensorView / nert::Attribute).
"""

from __future__ import annotations

import ctypes as C
from typing import Any, Iterable, Sequence

import numpy as np

F32, I64, BOOL, UNKNOWN = 0, 1, 2, 3
ATTR_INT, ATTR_FLOAT, ATTR_STRING, ATTR_INTS, ATTR_FLOATS, ATTR_BOOL = range(6)
OK, INFERENCE_ERROR, OTHER_ERROR, NO_KERNEL = range(4)

_NP_TO_CODE = {np.dtype(np.float32): F32, np.dtype(np.int64): I64, np.dtype(np.bool_): BOOL}
CODE_TO_NP = {F32: np.float32, I64: np.int64, BOOL: np.bool_}


class TensorDesc(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("rank", C.c_int32), ("dims", C.POINTER(C.c_int64))]


class AttrDesc(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("kind", C.c_int32),
        ("_pad", C.c_int32),
        ("i", C.c_int64),
        ("f", C.c_float),
        ("_pad2", C.c_int32),
        ("s", C.c_char_p),
        ("ints", C.POINTER(C.c_int64)),
        ("floats", C.POINTER(C.c_float)),
        ("count", C.c_int64),
    ]


def dtype_code(dtype: Any) -> int:
    return _NP_TO_CODE[np.dtype(dtype)]


class Float(float):
    """Marks a Python number as a FLOAT attribute even when it is integral."""


class AttrPack:
    """Owns the C storage behind an attribute array for one call."""

    def __init__(self, attrs: dict[str, Any] | None):
        attrs = attrs or {}
        self._keep: list[Any] = []
        self.array = (AttrDesc * max(1, len(attrs)))()
        self.count = len(attrs)
        for idx, (name, value) in enumerate(attrs.items()):
            d = self.array[idx]
            bname = name.encode()
            self._keep.append(bname)
            d.name = bname
            if isinstance(value, (bool, np.bool_)):
                d.kind, d.i = ATTR_BOOL, int(bool(value))
            elif isinstance(value, Float) or isinstance(value, (float, np.floating)):
                d.kind, d.f = ATTR_FLOAT, float(value)
            elif isinstance(value, (int, np.integer)):
                d.kind, d.i = ATTR_INT, int(value)
            elif isinstance(value, str):
                b = value.encode()
                self._keep.append(b)
                d.kind, d.s = ATTR_STRING, b
            elif isinstance(value, (list, tuple, np.ndarray)):
                vals = list(value)
                if vals and all(isinstance(v, (float, np.floating)) for v in vals):
                    arr = (C.c_float * len(vals))(*vals)
                    d.kind, d.floats, d.count = ATTR_FLOATS, C.cast(arr, C.POINTER(C.c_float)), len(vals)
                else:
                    arr = (C.c_int64 * max(1, len(vals)))(*[int(v) for v in vals])
                    d.kind, d.ints, d.count = ATTR_INTS, C.cast(arr, C.POINTER(C.c_int64)), len(vals)
                self._keep.append(arr)
            else:
                raise TypeError(f"unsupported attribute {name}={value!r}")


class TensorPack:
    """Owns the dims storage of a tensor-description array for one call.

    Each entry is None (an omitted optional operand) or a tuple
    (data pointer, dtype code, dims)."""

    def __init__(self, entries: Sequence[tuple[int, int, Sequence[int]] | None]):
        self._keep: list[Any] = []
        self.count = len(entries)
        self.array = (TensorDesc * max(1, len(entries)))()
        for idx, e in enumerate(entries):
            d = self.array[idx]
            if e is None:
                d.data, d.dtype, d.rank, d.dims = None, UNKNOWN, -1, None
                continue
            ptr, code, dims = e
            dims_arr = (C.c_int64 * max(1, len(dims)))(*[int(x) for x in dims])
            self._keep.append(dims_arr)
            d.data, d.dtype, d.rank = ptr, code, len(dims)
            d.dims = C.cast(dims_arr, C.POINTER(C.c_int64))


def host_entries(arrays: Iterable[np.ndarray | None]) -> list[tuple[int, int, Sequence[int]] | None]:
    out: list[tuple[int, int, Sequence[int]] | None] = []
    for a in arrays:
        if a is None:
            out.append(None)
            continue
        if not (isinstance(a, np.ndarray) and a.flags.c_contiguous):
            raise TypeError("host tensors must be C-contiguous numpy arrays")
        ptr = a.ctypes.data if a.size > 0 else 0
        out.append((ptr, dtype_code(a.dtype), a.shape))
    return out


def node_argtypes() -> list[Any]:
    return [C.c_char_p, C.c_char_p, C.c_int64, C.POINTER(AttrDesc), C.c_int, C.POINTER(TensorDesc), C.c_int,
            C.POINTER(TensorDesc), C.c_int, C.c_char_p, C.c_int]
