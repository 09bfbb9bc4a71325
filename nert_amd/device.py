"""Python host side of the gfx950 device layer (ctypes over include/nert_hip.h).

Mirrors how the reference drives a device through its seam: device buffers
come from the layer's allocator, tensors move with blocking transfers, and a
node runs through `run_node`, the C form of
`HipDevice().kernels().find(op)(node, inputs, outputs)`
(include/nert/device.hpp:30-31,96; src/executor.cpp:534).

There is no fallback: if nert_amd/lib/libnert_hip.so is missing or no GPU is
usable, every entry point raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from . import abi

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libnert_hip.so"


class NertError(RuntimeError):
    """A row or runtime failure; `status` is a nert_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.message = message


_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NertError(abi.OTHER_ERROR, f"{LIB_PATH} is not built; run `python -m nert_amd.build`")
    L = C.CDLL(str(LIB_PATH))
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
    L.nert_hip_last_error.restype = C.c_char_p
    L.nert_hip_malloc.restype = vp
    L.nert_hip_malloc.argtypes = [i64]
    L.nert_hip_free.argtypes = [vp]
    L.nert_hip_host_alloc.restype = vp
    L.nert_hip_host_alloc.argtypes = [i64]
    L.nert_hip_host_free.argtypes = [vp]
    L.nert_hip_memcpy_h2d.argtypes = [vp, vp, i64]
    L.nert_hip_memcpy_d2h.argtypes = [vp, vp, i64]
    L.nert_hip_memcpy_d2d.argtypes = [vp, vp, i64, vp]
    L.nert_hip_default_stream.restype = vp
    L.nert_hip_stream_sync.argtypes = [vp]
    L.nert_hip_event_create.restype = vp
    L.nert_hip_event_record.argtypes = [vp, vp]
    L.nert_hip_event_elapsed_ms.argtypes = [vp, vp, C.POINTER(C.c_float)]
    L.nert_hip_event_destroy.argtypes = [vp]
    L.nert_hip_run_node.argtypes = abi.node_argtypes()
    L.nert_hip_has_row.argtypes = [C.c_char_p]
    L.nert_hip_gemm_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i32, C.c_float, C.c_float, i32, vp]
    L.nert_hip_matmul_f32.argtypes = [vp, vp, vp, i64, i64, i64, i32, vp, vp, vp, vp]
    L.nert_hip_conv_f32.argtypes = [vp, vp, vp, vp, vp, vp]
    L.nert_hip_unary.argtypes = [i32, i32, vp, vp, i64, C.c_double, C.c_double, vp]
    L.nert_hip_capture_end.argtypes = [C.POINTER(C.c_void_p)]
    L.nert_hip_graph_launch.argtypes = [vp, vp]
    L.nert_hip_graph_destroy.argtypes = [vp]
    L.nert_hip_take_error_flags.argtypes = [C.POINTER(C.c_int32), vp]
    L.nert_hip_gather.argtypes = [i32, vp, vp, vp, i64, i64, i64, i64, vp]
    L.nert_hip_attention_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, C.POINTER(C.c_int64),
                                         C.POINTER(C.c_int64), C.c_float, vp]
    _lib = L
    return L


def last_error() -> str:
    msg = lib().nert_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise NertError(abi.OTHER_ERROR, f"{what}: {last_error()}")


def init() -> None:
    check(lib().nert_hip_init(), "nert_hip_init")


def synchronize() -> None:
    check(lib().nert_hip_stream_sync(None), "nert_hip_stream_sync")


ERROR_FLAG_TEXT = {1: "integer division by zero", 2: "index out of range"}


def take_error_flags() -> int:
    """Reads and clears the device error word (synchronises the layer
    stream): bit 0 integer division by zero, bit 1 index out of range."""
    flags = C.c_int32(0)
    check(lib().nert_hip_take_error_flags(C.byref(flags), None), "nert_hip_take_error_flags")
    return int(flags.value)


class PinnedArray:
    """A numpy array over pinned host memory (nert_hip_host_alloc): copies
    to and from it go straight to the DMA engine, with no bounce buffer."""

    def __init__(self, shape: Sequence[int], dtype: Any):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = lib().nert_hip_host_alloc(self.nbytes) if self.nbytes > 0 else None
        if self.nbytes > 0 and not self.ptr:
            raise NertError(abi.OTHER_ERROR, f"nert_hip_host_alloc({self.nbytes}): {last_error()}")
        if self.ptr:
            raw = (C.c_uint8 * self.nbytes).from_address(self.ptr)
            self.array = np.frombuffer(raw, np.uint8).view(self.dtype).reshape(self.shape)
        else:
            self.array = np.empty(self.shape, self.dtype)

    def close(self) -> None:
        if self.ptr:
            self.array = None
            lib().nert_hip_host_free(self.ptr)
            self.ptr = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class DeviceArray:
    """A device tensor allocated by the layer (freed on close / collection)."""

    def __init__(self, shape: Sequence[int], dtype: Any):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = lib().nert_hip_malloc(self.nbytes) if self.nbytes > 0 else None
        if self.nbytes > 0 and not self.ptr:
            raise NertError(abi.OTHER_ERROR, f"nert_hip_malloc({self.nbytes}): {last_error()}")

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.asarray(a, order="C")  # keeps 0-d arrays 0-d
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(lib().nert_hip_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes), "h2d")
        return d

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().nert_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes), "d2h")
        return out

    def close(self) -> None:
        if self.ptr:
            lib().nert_hip_free(self.ptr)
            self.ptr = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    @property
    def entry(self) -> tuple[int, int, Sequence[int]]:
        return (self.ptr or 0, abi.dtype_code(self.dtype), self.shape)


def has_row(op_type: str) -> bool:
    return bool(lib().nert_hip_has_row(op_type.encode()))


def run_node(op_type: str, inputs: Sequence[DeviceArray | None], outputs: Sequence[DeviceArray],
             attrs: dict[str, Any] | None = None, name: str = "n", schema_version: int = 0) -> None:
    """Runs one HIP row; raises NertError with the row's message on failure."""
    ap = abi.AttrPack(attrs)
    ip = abi.TensorPack([None if t is None else t.entry for t in inputs])
    op = abi.TensorPack([t.entry for t in outputs])
    err = C.create_string_buffer(4096)
    rc = lib().nert_hip_run_node(op_type.encode(), name.encode(), schema_version, ap.array, ap.count, ip.array,
                                 ip.count, op.array, op.count, err, len(err))
    if rc != abi.OK:
        raise NertError(rc, err.value.decode())


class Event:
    def __init__(self) -> None:
        self.ptr = lib().nert_hip_event_create()
        if not self.ptr:
            raise NertError(abi.OTHER_ERROR, f"event create: {last_error()}")

    def record(self, stream: int | None = None) -> None:
        check(lib().nert_hip_event_record(self.ptr, stream), "event record")

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float()
        check(lib().nert_hip_event_elapsed_ms(self.ptr, stop.ptr, C.byref(ms)), "event elapsed")
        return float(ms.value)

    def __del__(self) -> None:
        try:
            if self.ptr:
                lib().nert_hip_event_destroy(self.ptr)
        except Exception:
            pass


def gpu_available() -> bool:
    """True when the library loads and a HIP device initialises."""
    if os.environ.get("NERT_FORCE_NO_GPU") == "1":
        return False
    try:
        return lib().nert_hip_init() == 0
    except (OSError, NertError):
        return False
