"""CPU: the C-ABI library loads and exports every entry point include/*.h
declares; the HIP table has a row wherever the reference CPU table does.
No compute calls (there is no GPU here)."""

import ctypes
import re
from pathlib import Path

import pytest

from nert_amd import device
from oracle import ref

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s]*?[\s\*]+(nert_\w+)\s*\(", re.M)

# The reference CPU table (src/kernels/cpu_kernels.cpp:15-93).
REFERENCE_ROWS = [
    "Relu", "Add", "Mul", "Div", "Sub", "Sigmoid", "Cast", "Softmax", "ReduceMax", "Mod", "Equal", "Greater",
    "Less", "And", "Not", "Where", "Reshape", "ReduceMean", "Gemm", "MatMul", "Conv", "MaxPool", "Concat", "Split",
    "Unsqueeze", "Expand", "Transpose", "Slice", "Gather", "GatherElements", "Resize", "Flatten", "Shape",
    "ConstantOfShape", "TopK", "Floor", "Identity", "Pow", "Abs", "Neg", "Sign", "Exp", "Log", "Cos", "Sin", "Clip",
    "Tile", "AveragePool", "GlobalAveragePool", "GridSample", "Einsum", "ConvTranspose", "Erf", "Sqrt", "Tanh",
    "IsNaN", "Squeeze", "LayerNormalization", "InstanceNormalization", "ReduceSum", "Range", "Pad", "Elu", "Max",
    "Min", "LessOrEqual", "GreaterOrEqual", "Or", "ReduceL2", "ArgMax", "CumSum", "EyeLike", "ScatterND",
]


def declared_symbols():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(DECL.findall(text))
    return sorted(names)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "nert_hip_gemm_f32" in syms and "nert_hip_run_node" in syms and "nert_hip_conv_f32" in syms


@pytest.mark.parametrize("name", declared_symbols())
def test_library_exports(name):
    lib = ctypes.CDLL(str(device.LIB_PATH))
    assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_reference_table_is_73_rows():
    assert len(REFERENCE_ROWS) == 73 and len(set(REFERENCE_ROWS)) == 73
    assert all(ref.has_row(op) for op in REFERENCE_ROWS)
    assert not ref.has_row("BatchNormalization")


def test_hip_table_rows():
    """Every reference row has a HIP row, plus the runner's internal fused
    rows FusedConv, FusedMatMul, FusedAddLayerNorm and FusedAttention (lookup
    only; no device call)."""
    missing = [op for op in REFERENCE_ROWS if not device.has_row(op)]
    assert missing == [], f"rows without a HIP kernel: {missing}"
    assert device.has_row("FusedConv")
    assert device.has_row("FusedMatMul")
    assert device.has_row("FusedAddLayerNorm")
    assert device.has_row("FusedAttention")
    assert not device.has_row("BatchNormalization")
    assert not device.has_row("")


def test_hip_device_without_gpu_throws_inference_exception():
    """HipDevice() throws nert::InferenceException when no GPU is usable
    (src/hip_device.cpp:33-44; test/device_test_helpers.hpp:22-29 treats that
    as the device being absent). This container has no GPU."""
    import os

    from nert_amd import abi as _abi

    if device.gpu_available() and os.environ.get("NERT_FORCE_NO_GPU") != "1":
        pytest.skip("a GPU is present: the no-device path cannot be observed here")
    lib = ctypes.CDLL(str(ROOT / "tests" / "_build" / "libnert_contract.so"))
    name = ctypes.create_string_buffer(64)
    is_host, offsets = ctypes.c_int(), ctypes.c_int()
    err = ctypes.create_string_buffer(1024)
    rc = lib.contract_device_facts(name, 64, ctypes.byref(is_host), ctypes.byref(offsets), err, 1024)
    assert rc == _abi.INFERENCE_ERROR, (rc, err.value)
    assert err.value.decode(), "the exception names its cause"
