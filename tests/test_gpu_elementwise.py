"""GPU parity: unary, broadcast, comparison/logic, Where, Cast, Clip, pooling
and copy rows against the reference CpuDevice rows."""

import numpy as np
import pytest

from rowcheck import assert_parity, assert_same_error, randn, rng, run_hip, run_ref

pytestmark = pytest.mark.gpu

F, I, B = np.float32, np.int64, np.bool_

SPECIAL = np.array([0.0, -0.0, 1.5, -2.25, np.inf, -np.inf, np.nan, 1e-30, -1e30, 88.0, -88.0], F)

FLOAT_UNARY = ["Relu", "Sigmoid", "Tanh", "Exp", "Sqrt", "Sin", "Cos", "Floor", "Erf", "Abs", "Neg", "Sign", "Elu"]


@pytest.mark.parametrize("op", FLOAT_UNARY + ["Log"])
def test_unary_float(gpu, op):
    x = randn((3, 5, 37), seed=1, scale=2.0)
    if op in ("Sqrt", "Log"):
        x = np.abs(x) + F(0.01)
    assert_parity(op, [x], [(x.shape, F)])


@pytest.mark.parametrize("op", FLOAT_UNARY)
def test_unary_special_values(gpu, op):
    assert_parity(op, [SPECIAL], [(SPECIAL.shape, F)])


def test_unary_large_vectorized(gpu):
    x = randn((4, 1 << 20), seed=2)
    assert_parity("Relu", [x], [(x.shape, F)])
    x2 = randn((1000003,), seed=3)  # odd length: vector body + scalar tail
    assert_parity("Sigmoid", [x2], [(x2.shape, F)])


@pytest.mark.parametrize("op", ["Abs", "Neg", "Sign"])
def test_unary_int64(gpu, op):
    x = np.array([0, 1, -1, 7, -9, 2**40, -(2**40), 2**63 - 1, -(2**63) + 1], I)
    assert_parity(op, [x], [(x.shape, I)])


def test_sign_int64_extremes(gpu):
    """Sign over the whole int64 range, INT64_MIN included: the reference's
    cross-device release contract (test/release_kernels_test.cpp:41-46)."""
    x = np.array([np.iinfo(I).min, -1, 0, 1, np.iinfo(I).max], I)
    got = assert_parity("Sign", [x], [(x.shape, I)])
    assert np.array_equal(got[0], np.array([-1, -1, 0, 1, 1], I))


def test_elu_alpha(gpu):
    x = randn((1000,), seed=4)
    assert_parity("Elu", [x], [(x.shape, F)], {"alpha": 0.3})


def test_isnan_not(gpu):
    assert_parity("IsNaN", [SPECIAL], [(SPECIAL.shape, B)])
    m = rng(5).integers(0, 2, (7, 9)).astype(B)
    assert_parity("Not", [m], [(m.shape, B)])


def test_clip_variants(gpu):
    x = np.concatenate([SPECIAL, randn((50,), seed=6, scale=3)])
    assert_parity("Clip", [x], [(x.shape, F)])
    assert_parity("Clip", [x, np.array(-1.0, F), np.array(2.0, F)], [(x.shape, F)])
    assert_parity("Clip", [x, None, np.array(0.5, F)], [(x.shape, F)])
    xi = np.arange(-10, 10, dtype=I)
    assert_parity("Clip", [xi, np.array(-3, I), np.array(4, I)], [(xi.shape, I)])
    assert_parity("Clip", [xi, np.array(-(2**63), I)], [(xi.shape, I)])


BROADCASTS = [
    ((4, 8, 16), (4, 8, 16)),
    ((32, 64, 7, 7), (64, 1, 1)),
    ((16, 197, 768), (768,)),
    ((2, 3, 1, 5), (1, 1, 4, 1)),
    ((5,), ()),
    ((), (3, 4)),
    ((16, 197, 64), ()),       # scalar operand: one-row rank-2 walk
    ((), (2, 3, 8)),
    ((1, 1, 4096), (1,)),
    ((3, 1), (1, 4)),
    ((2, 1, 3, 1, 4, 1, 2), (1, 5, 1, 6, 1, 7, 1)),
]


@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div", "Pow", "Max", "Min"])
@pytest.mark.parametrize("sa,sb", BROADCASTS)
def test_binary_float_broadcast(gpu, op, sa, sb):
    a = randn(sa, seed=7)
    b = randn(sb, seed=8)
    if op == "Pow":
        a = np.abs(a) + F(0.1)
    out = np.broadcast_shapes(sa, sb)
    assert_parity(op, [a, b], [(out, F)])


def test_binary_float_specials(gpu):
    a = np.repeat(SPECIAL, len(SPECIAL))
    b = np.tile(SPECIAL, len(SPECIAL))
    for op in ["Add", "Sub", "Mul", "Div", "Max", "Min", "Pow"]:
        assert_parity(op, [a, b], [(a.shape, F)])
    assert_parity("Pow", [randn((64,), seed=9), np.array(2.0, F)], [((64,), F)])


@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div", "Max", "Min", "Mod"])
def test_binary_int64(gpu, op):
    a = rng(10).integers(-1000, 1000, (6, 5)).astype(I)
    b = rng(11).integers(1, 50, (5,)).astype(I) * rng(12).choice([-1, 1], (5,))
    assert_parity(op, [a, b], [((6, 5), I)])


@pytest.mark.parametrize("op", ["Div", "Mod"])
def test_int64_division_by_zero_throws(gpu, op):
    a = np.array([4, 5, 6], I)
    b = np.array([1, 0, 2], I)
    msg = assert_same_error(op, [a, b], [((3,), I)])
    assert "division by zero" in msg


@pytest.mark.parametrize("op", ["Div", "Mod"])
def test_int64_division_by_zero_device_checked(gpu, op):
    """A divisor above the 64 KiB host-shadow limit is checked by the kernel's
    error flag instead of on the host: same exception."""
    a = rng(13).integers(-1000, 1000, (9000,)).astype(I)
    b = rng(14).integers(1, 50, (9000,)).astype(I)
    b[8765] = 0
    msg = assert_same_error(op, [a, b], [((9000,), I)])
    assert "division by zero" in msg
    b[8765] = 3
    assert_parity(op, [a, b], [((9000,), I)])


def test_float_division_by_zero_is_ieee(gpu):
    a = np.array([1, -1, 0], F)
    b = np.zeros(3, F)
    assert_parity("Div", [a, b], [((3,), F)])


@pytest.mark.parametrize("op", ["Equal", "Greater", "Less", "GreaterOrEqual", "LessOrEqual"])
def test_compare(gpu, op):
    a = rng(13).integers(-3, 3, (4, 1, 6)).astype(F)
    b = rng(14).integers(-3, 3, (5, 1)).astype(F)
    assert_parity(op, [a, b], [((4, 5, 6), B)])
    ai = rng(15).integers(-3, 3, (7,)).astype(I)
    bi = rng(16).integers(-3, 3, (7,)).astype(I)
    assert_parity(op, [ai, bi], [((7,), B)])
    assert_parity(op, [SPECIAL, SPECIAL[::-1].copy()], [(SPECIAL.shape, B)])


@pytest.mark.parametrize("op", ["And", "Or"])
def test_logic(gpu, op):
    a = rng(17).integers(0, 2, (3, 4)).astype(B)
    b = rng(18).integers(0, 2, (4,)).astype(B)
    assert_parity(op, [a, b], [((3, 4), B)])


def test_where(gpu):
    c = rng(19).integers(0, 2, (3, 1, 5)).astype(B)
    x = randn((4, 5), seed=20)
    y = randn((3, 4, 1), seed=21)
    assert_parity("Where", [c, x, y], [((3, 4, 5), F)])
    xi = rng(22).integers(-9, 9, (5,)).astype(I)
    yi = rng(23).integers(-9, 9, (3, 1, 1)).astype(I)
    assert_parity("Where", [c, xi, yi], [((3, 1, 5), I)])


def test_max_min_variadic(gpu):
    a, b, c = randn((3, 4), seed=24), randn((4,), seed=25), randn((2, 1, 4), seed=26)
    for op in ["Max", "Min"]:
        assert_parity(op, [a], [((3, 4), F)])
        assert_parity(op, [a, b, c], [((2, 3, 4), F)])
    nan_first = np.array([np.nan, 1.0, 2.0], F)
    assert_parity("Max", [nan_first, np.array([0.0, np.nan, 5.0], F)], [((3,), F)])


@pytest.mark.parametrize("to,src", [(1, I), (1, B), (7, F), (6, F), (9, F), (9, I), (6, I), (7, B), (1, F)])
def test_cast(gpu, to, src):
    vals = np.array([0.0, -0.0, 1.0, -1.7, 2.5, 3e9, -3e9, 1e20, np.nan, np.inf, 0.3], np.float64)
    x = vals.astype(src) if src != I else np.array([0, 1, -5, 2**40, 2**31, -(2**31) - 5, 7], I)
    if src == B:
        x = np.array([0, 1, 1, 0], B)
    if src == F and to == 7:
        x = np.array([0.0, -0.0, 1.0, -1.7, 2.5, 3e9, -3e9, 0.3, -123456.7], F)  # in-range only: UB otherwise
    dst = {1: F, 6: I, 7: I, 9: B}[to]
    assert_parity("Cast", [x], [(x.shape, dst)], {"to": to})


def test_error_messages(gpu):
    assert_same_error("Add", [randn((2, 3)), randn((4,))], [((2, 3), F)])
    assert_same_error("Relu", [randn((2, 3))], [((2, 3), I)])
    assert_same_error("Where", [randn((2,)), randn((2,)), randn((2,))], [((2,), F)])


# --- pools ----------------------------------------------------------------

POOL_CASES = [
    ((32, 64, 112, 112), {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]}),
    ((2, 3, 10, 11), {"kernel_shape": [2, 3], "strides": [2, 1]}),
    ((1, 2, 9, 9), {"kernel_shape": [3, 3], "strides": [2, 2], "ceil_mode": 1}),
    ((1, 2, 9, 9), {"kernel_shape": [2, 2], "auto_pad": "SAME_UPPER", "strides": [2, 2]}),
    ((1, 2, 9, 9), {"kernel_shape": [3, 3], "dilations": [2, 2], "pads": [2, 2, 2, 2]}),
    ((2, 3, 30, 2000), {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}),  # wide rows: 4-row LDS tiles
    ((1, 1, 5, 5000), {"kernel_shape": [3, 3]}),                          # too wide for LDS: direct kernel
    ((1, 2, 20, 20), {"kernel_shape": [3, 3], "dilations": [2, 2], "pads": [2, 2, 2, 2]}),  # 4 outputs/thread
    ((1, 3, 17, 17), {"kernel_shape": [3, 3], "strides": [2, 2], "ceil_mode": 1}),         # ragged last window
    ((8, 64, 112, 112), {"kernel_shape": [3, 3], "strides": [2, 2]}),     # the reference bench case (55 wide)
]


def _pool_out(xs, a, dil=True):
    k, s = a["kernel_shape"], a.get("strides", [1, 1])
    d = a.get("dilations", [1, 1]) if dil else [1, 1]
    p = a.get("pads", [0, 0, 0, 0])
    if a.get("auto_pad") == "SAME_UPPER":
        return xs[:2] + tuple(-(-xs[2 + i] // s[i]) for i in range(2))
    out = []
    for i in range(2):
        num = xs[2 + i] + p[i] + p[i + 2] - (d[i] * (k[i] - 1) + 1)
        out.append((-(-num // s[i]) if a.get("ceil_mode") else num // s[i]) + 1)
    return xs[:2] + tuple(out)


@pytest.mark.parametrize("xs,attrs", POOL_CASES)
def test_maxpool(gpu, xs, attrs):
    x = randn(xs, seed=27)
    assert_parity("MaxPool", [x], [(_pool_out(xs, attrs), F)], attrs)


@pytest.mark.parametrize("xs,attrs", [c for c in POOL_CASES if "dilations" not in c[1]])
@pytest.mark.parametrize("include_pad", [0, 1])
def test_avgpool(gpu, xs, attrs, include_pad):
    x = randn(xs, seed=28)
    a = dict(attrs, count_include_pad=include_pad)
    assert_parity("AveragePool", [x], [(_pool_out(xs, a, dil=False), F)], a, rtol=0, atol=0)


def test_maxpool_nan_and_neg_inf(gpu):
    x = np.full((1, 1, 4, 4), np.nan, F)
    x[0, 0, 0, 0] = -np.inf
    assert_parity("MaxPool", [x], [((1, 1, 2, 2), F)], {"kernel_shape": [2, 2], "strides": [2, 2]})


@pytest.mark.parametrize("xs", [(32, 64, 112, 112), (3, 5, 7, 8), (2, 3, 20, 256), (1, 7, 33, 4), (2, 2, 1, 12),
                                (8, 64, 112, 112), (2, 3, 9, 12)])
@pytest.mark.parametrize("pad,ceil", [(1, 0), (0, 0), (0, 1)])
def test_maxpool_3x3_stride2_kernel(gpu, xs, pad, ceil):
    """The 3x3 / stride-2 pool from registers (one lane per column quad, rows
    reduced in registers): pad 1 (the ResNet stem pool), pad 0 (odd and even
    output widths; the reference's [8,64,112,112] fixture) and pad 0 in
    ceil mode (a right and bottom padding tap), over whole and partial row
    runs and one to 64 planes per wave: bit-identical to the reference, with
    signed zeros, NaNs and -inf sprinkled in."""
    if pad == 0 and xs[2] < 3:
        pytest.skip("no 3x3 window fits without padding")
    x = randn(xs, seed=31)
    flat = x.reshape(-1)
    pick = rng(32).random(flat.size)
    flat[pick < 0.05] = 0.0
    flat[(pick >= 0.05) & (pick < 0.1)] = -0.0
    flat[(pick >= 0.1) & (pick < 0.12)] = np.nan
    flat[(pick >= 0.12) & (pick < 0.13)] = -np.inf
    attrs = {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [pad] * 4, "ceil_mode": ceil}
    spec = [(_pool_out(xs, attrs), F)]
    want, ref_err = run_ref("MaxPool", [x], spec, attrs)
    got, hip_err = run_hip("MaxPool", [x], spec, attrs)
    assert ref_err is None and hip_err is None, (ref_err, hip_err)
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))


@pytest.mark.parametrize("xs", [(32, 512, 7, 7), (8, 64, 112, 112), (2, 3, 5), (1, 4, 2, 3, 4), (3, 5),
                                (2, 3, 47, 49), (1, 2, 4096, 1)])
def test_global_average_pool(gpu, xs):
    x = randn(xs, seed=29)
    out = xs[:2] + (1,) * (len(xs) - 2)
    assert_parity("GlobalAveragePool", [x], [(out, F)])


# --- copies ---------------------------------------------------------------

def test_identity_flatten_reshape(gpu):
    x = randn((2, 3, 4, 5), seed=30)
    assert_parity("Identity", [x], [(x.shape, F)])
    assert_parity("Flatten", [x], [((2, 60), F)])
    # the reference maps a negative axis to axis + rank + 1 (src/kernels/flatten.cpp:55-57)
    assert_parity("Flatten", [x], [((120, 1), F)], {"axis": -1})
    assert_parity("Flatten", [x], [((24, 5), F)], {"axis": -2})
    assert_parity("Flatten", [x], [((1, 120), F)], {"axis": 0})
    assert_parity("Reshape", [x, np.array([0, -1, 5], I)], [((2, 12, 5), F)])
    assert_parity("Reshape", [x, np.array([6, 20], I)], [((6, 20), F)])
    xi = np.arange(24, dtype=I).reshape(2, 12)
    assert_parity("Reshape", [xi, np.array([4, -1], I)], [((4, 6), I)])
    assert_same_error("Reshape", [x, np.array([7, -1], I)], [((7, 17), F)])
    assert_same_error("Flatten", [x], [((2, 61), F)])
