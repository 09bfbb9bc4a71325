"""GPU parity: index and generator rows (Gather, GatherElements, ScatterND,
Shape, ConstantOfShape, Range, EyeLike) against the reference CpuDevice rows.

Out-of-range indices must throw the reference's message on both routes the
HIP rows take: indices uploaded from the host (checked from the host shadow
before launch; uploads up to 64 KiB) and larger index tensors (checked by the
kernel's device flag)."""

import numpy as np
import pytest

from rowcheck import assert_parity, assert_same_error, randn, rng

pytestmark = pytest.mark.gpu

F, I, B = np.float32, np.int64, np.bool_
EXACT = {"rtol": 0.0, "atol": 0.0}
BIG = 10000  # 80 KB of int64 indices: beyond the host-shadow limit


def _data(shape, dtype, seed=0):
    if dtype == F:
        return randn(shape, seed=seed)
    if dtype == I:
        return rng(seed).integers(-1 << 40, 1 << 40, shape).astype(I)
    return rng(seed).integers(0, 2, shape).astype(B)


def _gather_shape(shape, idx_shape, axis):
    axis %= len(shape)
    return tuple(shape[:axis]) + tuple(idx_shape) + tuple(shape[axis + 1:])


@pytest.mark.parametrize("dtype", [F, I, B])
@pytest.mark.parametrize("shape,idx,axis", [
    ((16, 197, 768), np.array(0, I), 1),                 # ViT class token
    ((8, 8400, 4), rng(1).integers(-8400, 8400, (300,)).astype(I), 1),
    ((5, 6, 7), np.array([[0, -1], [4, 2]], I), 0),
    ((5, 6, 7), np.array([6, 0, -7], I), -1),
    ((1000, 3), rng(2).integers(-1000, 1000, (BIG,)).astype(I), 0),
    ((4, 5), np.zeros((0,), I), 1),
])
def test_gather(gpu, dtype, shape, idx, axis):
    x = _data(shape, dtype, seed=3)
    assert_parity("Gather", [x, idx], [(_gather_shape(shape, idx.shape, axis), dtype)], {"axis": axis}, **EXACT)


def test_gather_out_of_range(gpu):
    x = randn((6, 5))
    assert_same_error("Gather", [x, np.array([0, 6], I)], [((2, 5), F)])
    assert_same_error("Gather", [x, np.array([-6, 0], I)], [((6, 2), F)], {"axis": 1})
    big = rng(4).integers(0, 6, (BIG,)).astype(I)
    big[7777] = 6
    assert_same_error("Gather", [x, big], [((BIG, 5), F)])
    big[7777] = -7
    assert_same_error("Gather", [x, big], [((BIG, 5), F)])
    # the error flag is consumed: the next good call passes
    big[7777] = 1
    assert_parity("Gather", [x, big], [((BIG, 5), F)], **EXACT)
    # nothing is checked when the outer extent is empty (src/kernels/gather.cpp:31)
    assert_parity("Gather", [np.zeros((0, 5), F), np.array([9], I)], [((0, 1), F)], {"axis": 1})
    assert_same_error("Gather", [x, np.array([0.0], F)], [((1, 5), F)])
    assert_same_error("Gather", [x, np.array([0], I)], [((1, 6), F)])
    assert_same_error("Gather", [x, np.array([0], I)], [((1, 5), F)], {"axis": 2})


@pytest.mark.parametrize("dtype", [F, I])
@pytest.mark.parametrize("shape,idx_shape,axis", [
    ((4, 5, 6), (4, 3, 6), 1), ((4, 5, 6), (2, 5, 6), 0), ((4, 5, 6), (4, 5, 9), -1), ((7,), (12,), 0),
    ((3, 4), (2, 3), 1), ((100, 100), (100, 100), 0),
])
def test_gather_elements(gpu, dtype, shape, idx_shape, axis):
    x = _data(shape, dtype, seed=5)
    dim = shape[axis]
    idx = rng(6).integers(-dim, dim, idx_shape).astype(I)
    assert_parity("GatherElements", [x, idx], [(idx_shape, dtype)], {"axis": axis}, **EXACT)


def test_gather_elements_errors(gpu):
    x = randn((4, 5))
    assert_same_error("GatherElements", [x, np.array([[5]], I)], [((1, 1), F)])
    assert_same_error("GatherElements", [x, np.zeros((5, 1), I)], [((5, 1), F)])
    idx = rng(7).integers(0, 5, (4, 3000)).astype(I)  # 96 KB: device-checked
    idx[3, 2999] = -6
    assert_same_error("GatherElements", [randn((4, 5)), idx], [((4, 3000), F)])
    idx[3, 2999] = -5
    assert_parity("GatherElements", [randn((4, 5)), idx], [((4, 3000), F)], **EXACT)
    assert_same_error("GatherElements", [x.astype(B), np.zeros((4, 1), I)], [((4, 1), B)])


@pytest.mark.parametrize("dtype", [F, I, B])
def test_scatter_nd(gpu, dtype):
    data = _data((4, 5, 6), dtype, seed=8)
    # k = 1: whole [5, 6] slices, with duplicates (last wins) and negatives
    idx = np.array([[1], [-1], [1], [0]], I)
    upd = _data((4, 5, 6), dtype, seed=9)
    assert_parity("ScatterND", [data, idx, upd], [((4, 5, 6), dtype)], **EXACT)
    # k = 2: rows
    idx = np.array([[[0, 1], [3, -2]], [[0, 1], [2, 4]]], I)
    upd = _data((2, 2, 6), dtype, seed=10)
    assert_parity("ScatterND", [data, idx, upd], [((4, 5, 6), dtype)], **EXACT)
    # k = rank: single elements, many duplicates
    idx = rng(11).integers(-2, 2, (500, 3)).astype(I)
    upd = _data((500,), dtype, seed=12)
    assert_parity("ScatterND", [data, idx, upd], [((4, 5, 6), dtype)], **EXACT)


def test_scatter_nd_large_and_errors(gpu):
    data = randn((3000, 8))
    idx = rng(13).integers(0, 3000, (6000, 1)).astype(I)  # 48 KB
    upd = randn((6000, 8), seed=14)
    assert_parity("ScatterND", [data, idx, upd], [((3000, 8), F)], **EXACT)
    idx = rng(15).integers(-3000, 3000, (9000, 1)).astype(I)  # 72 KB: device-checked
    upd = randn((9000, 8), seed=16)
    assert_parity("ScatterND", [data, idx, upd], [((3000, 8), F)], **EXACT)
    idx[8000, 0] = 3000
    assert_same_error("ScatterND", [data, idx, upd], [((3000, 8), F)])
    assert_same_error("ScatterND", [data, np.array([[3000]], I), randn((1, 8))], [((3000, 8), F)])
    assert_same_error("ScatterND", [data, np.array([[0, 0, 0]], I), randn((1,))], [((3000, 8), F)])
    assert_same_error("ScatterND", [data, np.array([[0]], I), randn((1, 7))], [((3000, 8), F)])


def test_shape(gpu):
    x = randn((2, 3, 4, 5))
    assert_parity("Shape", [x], [((4,), I)], **EXACT)
    assert_parity("Shape", [x], [((2,), I)], {"start": 1, "end": -1}, **EXACT)
    assert_parity("Shape", [x], [((1,), I)], {"start": -1}, **EXACT)
    assert_parity("Shape", [x], [((0,), I)], {"start": 3, "end": 1}, **EXACT)
    assert_parity("Shape", [x.astype(B)], [((4,), I)], {"start": -10, "end": 10}, **EXACT)
    assert_parity("Shape", [np.array(1.0, F)], [((0,), I)], **EXACT)
    assert_same_error("Shape", [x], [((3,), I)])
    assert_same_error("Shape", [x], [((4,), F)])


def test_shape_feeds_control_reads(gpu):
    """Shape's output is read back by a later row (Reshape) without a device
    round trip; the values must be the ones the kernel writes."""
    from nert_amd.device import DeviceArray, run_node

    x = DeviceArray.from_host(randn((6, 4)))
    shp = DeviceArray.from_host(np.zeros((2,), I))
    run_node("Shape", [x], [shp], {}, "s")
    y = DeviceArray.from_host(np.zeros((6, 4), F))
    run_node("Reshape", [x, shp], [y], {}, "r")
    np.testing.assert_array_equal(shp.to_host(), [6, 4])
    np.testing.assert_array_equal(y.to_host(), x.to_host())


def test_constant_of_shape(gpu):
    assert_parity("ConstantOfShape", [np.array([2, 3], I)], [((2, 3), F)], **EXACT)
    assert_parity("ConstantOfShape", [np.array([4], I)], [((4,), F)], {"value": 2.5}, **EXACT)
    assert_parity("ConstantOfShape", [np.array([3, 1, 2], I)], [((3, 1, 2), I)], {"value": -7}, **EXACT)
    assert_parity("ConstantOfShape", [np.array([5], I)], [((5,), B)], {"value": True}, **EXACT)
    assert_parity("ConstantOfShape", [np.array([0, 3], I)], [((0, 3), F)], **EXACT)
    assert_parity("ConstantOfShape", [np.array([1 << 20], I)], [((1 << 20,), F)], {"value": 1.0}, **EXACT)
    assert_same_error("ConstantOfShape", [np.array([2], I)], [((2,), I)], {"value": 1.0})
    assert_same_error("ConstantOfShape", [np.array([-1], I)], [((1,), F)])
    assert_same_error("ConstantOfShape", [np.array([2], I)], [((3,), F)])


def test_range(gpu):
    def f(v):
        return np.array(v, F)

    def i(v):
        return np.array(v, I)

    def n(start, limit, delta):  # the length ONNX Range defines, from float32 operands
        return max(int(np.ceil((np.float64(f(limit)) - np.float64(f(start))) / np.float64(f(delta)))), 0)

    for start, limit, delta in [(0.5, 10.0, 0.3), (3.0, -4.0, -0.7), (1e6, 1e6 + 3e4, 0.37), (-2.0, 2.0, 0.1)]:
        assert_parity("Range", [f(start), f(limit), f(delta)], [((n(start, limit, delta),), F)], **EXACT)
    assert_parity("Range", [i(-5), i(100), i(7)], [((15,), I)], **EXACT)
    assert_parity("Range", [i(10), i(-10), i(-3)], [((7,), I)], **EXACT)
    assert_parity("Range", [i(10), i(1), i(1)], [((0,), I)], **EXACT)
    assert_same_error("Range", [i(0), i(10), i(0)], [((0,), I)])
    assert_same_error("Range", [i(0), i(10), i(3)], [((3,), I)])
    assert_same_error("Range", [f(0), i(10), f(3)], [((4,), F)])
    assert_same_error("Range", [f(0), f(10), np.array([1, 2], F)], [((4,), F)])


@pytest.mark.parametrize("dtype", [F, I, B])
def test_eye_like(gpu, dtype):
    for shape, k in [((4, 4), 0), ((3, 7), 2), ((6, 2), -3), ((5, 5), 9), ((300, 200), -1)]:
        assert_parity("EyeLike", [np.zeros(shape, F)], [(shape, dtype)], {"k": k}, **EXACT)
    assert_same_error("EyeLike", [np.zeros((2, 3, 4), F)], [((2, 3, 4), dtype)])


def _topk_case(x, k, axis=-1):
    out = list(x.shape)
    out[axis] = k
    out = tuple(out)
    assert_parity("TopK", [x, np.array(k, I)], [(out, F), (out, I)], {"axis": axis}, **EXACT)


@pytest.mark.parametrize("shape,k,axis", [
    ((2, 4), 2, -1), ((1000, 80), 5, 1), ((50, 7, 3), 4, 1), ((4096,), 4096, 0), ((3, 4097), 17, -1),
])
def test_topk_rows(gpu, shape, k, axis):
    _topk_case(randn(shape, seed=21), k, axis)
    ties = rng(22).integers(-3, 4, shape).astype(F)  # many equal values: index order decides
    _topk_case(ties, k, axis)


def test_topk_detector_shape(gpu):
    """The detector's score selection: [8, 672000] with K = 300 (radix select)."""
    x = randn((8, 672000), seed=23)
    _topk_case(x, 300)
    _topk_case(rng(24).integers(0, 50, (8, 672000)).astype(F), 300)  # ~13k-way ties per value


def test_topk_long_rows(gpu):
    _topk_case(randn((2, 20000), seed=25), 5000)       # sorted runs + merge passes
    _topk_case(randn((1, 9000), seed=26), 9000)        # K = dim on a long row
    _topk_case(randn((3, 6000, 2), seed=27), 100, 1)   # strided rows
    z = np.zeros((2, 10000), F)
    z[:, 1::2] = -0.0
    z[1, 7777] = 1e-30
    _topk_case(z, 64)                                   # -0.0 ties with +0.0


def test_topk_long_row_select_paths(gpu):
    """Long rows with K <= 1024 read the row once in chunks, and the row's
    last chunk workgroup merges the chunks' candidates; each of the merge's
    ways is exercised: the candidates from the chunks' lists or (past a
    list's capacity) from the row again, and the keys tied on 24 bits ranked
    in LDS or (past its capacity) radix-selected."""
    r = rng(31)
    _topk_case(randn((3, 50000), seed=32), 1)                        # K = 1
    _topk_case(randn((2, 70000), seed=33), 1024)                     # the largest K of this path
    spread = (1.0 + r.random((4, 100000)) * 0.125).astype(F)         # one 12-bit bin: the row reread, ranked ties
    _topk_case(spread, 300)
    same = np.full((2, 10000), 2.5, F)                               # one value: listed, radix-selected ties
    _topk_case(same, 100)
    inf = randn((2, 30000), seed=34)
    inf[0, ::1000] = np.inf
    inf[1, 5::777] = np.inf
    inf[1, 7] = -np.inf
    _topk_case(inf, 40)                                              # +inf ties, the top bin
    few = np.zeros((2, 40000), F)
    few[:, 123] = 1.0
    _topk_case(few, 300)                                             # one key above the threshold bin


_TWO_LAUNCH = """
import ctypes as C, sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd import device
from nert_amd.device import DeviceArray
device.init()
L = device.lib()
L.nert_hip_topk_f32.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 4 + [C.c_void_p]
out = {{}}
for name, (rows, dim, k, seed) in {cases!r}.items():
    x = np.load({path!r} + name + ".npy")
    dx = DeviceArray.from_host(x)
    v = DeviceArray((rows, k), np.float32)
    i = DeviceArray((rows, k), np.int64)
    assert L.nert_hip_topk_f32(dx.ptr, v.ptr, i.ptr, rows, dim, 1, k, None) == 0, device.last_error()
    device.synchronize()
    out[name + "_v"] = v.to_host()
    out[name + "_i"] = i.to_host()
np.savez({path!r} + "out.npz", **out)
"""


def test_topk_merge_in_chunk_launch_matches_two_launches(gpu, tmp_path):
    """The fused path (the row's last chunk workgroup merges, per-row
    counters) against the two-launch path (NERT_HIP_SPLIT_FIXUP=0, a merge
    launch of one workgroup per row) in a fresh process: bit-identical
    values and indices, twice in a row on the fused side (the counters are
    left zero)."""
    import ctypes as C
    import os
    import subprocess
    import sys

    from nert_amd import device
    from nert_amd.device import DeviceArray

    cases = {"det": (8, 672000, 300, 41), "ties": (5, 100000, 64, 42), "one": (3, 50000, 1, 43)}
    path = str(tmp_path) + os.sep
    xs = {}
    for name, (rows, dim, k, seed) in cases.items():
        r = rng(seed)
        x = r.random((rows, dim), dtype=np.float32)
        if name == "ties":
            x = r.integers(0, 20, (rows, dim)).astype(F)
        xs[name] = x
        np.save(path + name + ".npy", x)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, NERT_HIP_SPLIT_FIXUP="0")
    subprocess.run([sys.executable, "-c", _TWO_LAUNCH.format(root=root, cases=cases, path=path)], env=env,
                   check=True, timeout=120)
    want = np.load(path + "out.npz")
    L = device.lib()
    L.nert_hip_topk_f32.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 4 + [C.c_void_p]
    for _ in range(2):
        for name, (rows, dim, k, _seed) in cases.items():
            dx = DeviceArray.from_host(xs[name])
            v = DeviceArray((rows, k), np.float32)
            i = DeviceArray((rows, k), np.int64)
            assert L.nert_hip_topk_f32(dx.ptr, v.ptr, i.ptr, rows, dim, 1, k, None) == 0, device.last_error()
            device.synchronize()
            assert np.array_equal(v.to_host(), want[name + "_v"]), name
            assert np.array_equal(i.to_host(), want[name + "_i"]), name


def test_topk_errors(gpu):
    x = randn((3, 5))
    assert_same_error("TopK", [x, np.array(6, I)], [((3, 6), F), ((3, 6), I)])
    assert_same_error("TopK", [x, np.array(0, I)], [((3, 0), F), ((3, 0), I)])
    assert_same_error("TopK", [x, np.array(2, I)], [((3, 2), F), ((3, 2), I)], {"largest": 0})
    assert_same_error("TopK", [x, np.array(2, I)], [((3, 2), F), ((3, 2), I)], {"sorted": 0})
    assert_same_error("TopK", [x, np.array(2, I)], [((2, 5), F), ((2, 5), I)], {"axis": 2})
    assert_same_error("TopK", [x, np.array([2, 2], I)], [((3, 2), F), ((3, 2), I)])
