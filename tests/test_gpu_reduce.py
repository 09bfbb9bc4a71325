"""GPU parity: reduction rows (ReduceMean/Max/Sum/L2, Softmax, LayerNorm,
InstanceNorm, ArgMax, CumSum) against the reference CpuDevice rows, including
the schema-dependent operand forms (attribute axes before opset 18 for
ReduceMean/Max/L2 and before 13 for ReduceSum; Softmax's pre-13 2-D
coercion)."""

import numpy as np
import pytest

from rowcheck import assert_parity, assert_same_error, randn, rng

pytestmark = pytest.mark.gpu

F, I, B = np.float32, np.int64, np.bool_


def _reduced_shape(shape, axes, keepdims):
    axes = [a % len(shape) for a in axes] if axes else list(range(len(shape)))
    out = []
    for i, d in enumerate(shape):
        if i in axes:
            if keepdims:
                out.append(1)
        else:
            out.append(d)
    return tuple(out)


REDUCE_CASES = [
    ((32, 512, 7, 7), [2, 3], 1),
    ((16, 197, 768), [-1], 1),
    ((4, 5, 6), [0], 0),
    ((4, 5, 6), [1], 1),
    ((3, 4, 5, 6), [0, 2], 0),
    ((3, 4, 5, 6), [1, 3], 1),
    ((7, 9), [], 1),
    ((2, 3, 4), [0, 1, 2], 0),
]


@pytest.mark.parametrize("op", ["ReduceMean", "ReduceMax", "ReduceL2", "ReduceSum"])
@pytest.mark.parametrize("shape,axes,keepdims", REDUCE_CASES)
def test_reduce_input_form(gpu, op, shape, axes, keepdims):
    """Schema 0/18 form: axes as an int64 input (absent -> all axes)."""
    x = randn(shape, seed=len(shape))
    inputs = [x] if not axes else [x, np.array(axes, I)]
    out = _reduced_shape(shape, axes, keepdims)
    assert_parity(op, inputs, [(out, F)], {"keepdims": keepdims})


@pytest.mark.parametrize("op,schema", [("ReduceMean", 17), ("ReduceMax", 13), ("ReduceL2", 13), ("ReduceSum", 11)])
def test_reduce_attribute_form(gpu, op, schema):
    x = randn((6, 5, 4), seed=3)
    assert_parity(op, [x], [((6, 1, 4), F)], {"axes": [1], "keepdims": 1}, schema_version=schema)
    assert_parity(op, [x], [((), F)], {"keepdims": 0}, schema_version=schema)


def test_reduce_noop_and_special(gpu):
    x = randn((3, 4), seed=4)
    for op in ["ReduceMean", "ReduceL2", "ReduceSum"]:
        assert_parity(op, [x, np.zeros((0,), I)], [((3, 4), F)], {"noop_with_empty_axes": 1})
    xi = rng(5).integers(-1000, 1000, (5, 6)).astype(I)
    assert_parity("ReduceSum", [xi, np.array([1], I)], [((5, 1), I)])
    nan = np.array([[np.nan, 1.0, 2.0], [np.nan, np.nan, np.nan]], F)
    assert_parity("ReduceMax", [nan, np.array([1], I)], [((2, 1), F)])
    assert_same_error("ReduceMean", [x, np.array([0, 0], I)], [((1, 4), F)])
    assert_same_error("ReduceMax", [x, np.array([2], I)], [((3, 1), F)])


SOFTMAX_CASES = [((16, 12, 197, 197), -1), ((4, 4096), -1), ((3, 5, 7), 1), ((2, 3, 4), 0), ((1000,), 0),
                 ((7, 300), -1), ((5, 64), -1), ((9, 224), -1), ((3, 225), -1), ((11, 1), -1),
                 ((5, 2001), -1), ((3, 1028), -1), ((2, 4097), -1), ((256, 4096), -1)]  # workgroup-per-row paths


@pytest.mark.parametrize("shape,axis", SOFTMAX_CASES)
def test_softmax(gpu, shape, axis):
    x = randn(shape, seed=6, scale=3.0)
    assert_parity("Softmax", [x], [(shape, F)], {"axis": axis})


def test_softmax_legacy_and_specials(gpu):
    x = randn((2, 3, 4), seed=7)
    assert_parity("Softmax", [x], [((2, 3, 4), F)], schema_version=11)  # coerced 2-D, default axis 1
    assert_parity("Softmax", [x], [((2, 3, 4), F)], {"axis": 2}, schema_version=11)
    s = np.array([[np.nan, 1, 2], [1, np.nan, 3], [np.inf, 1, 2], [-np.inf, 0, 1], [1e30, 1e30, -1e30]], F)
    assert_parity("Softmax", [s], [(s.shape, F)])
    assert_same_error("Softmax", [x], [((2, 3, 4), F)], {"axis": 3})


@pytest.mark.parametrize("shape,axis", [((16, 197, 768), -1), ((4, 6, 10), 1), ((8, 33), 0), ((5, 1024), -1),
                                        ((3, 2000), -1), ((6, 256), -1)])
def test_layernorm(gpu, shape, axis):
    x = randn(shape, seed=8, scale=2.0) + 0.5
    ax = axis % len(shape)
    inner = int(np.prod(shape[ax:]))
    outer = int(np.prod(shape[:ax]))
    scale = randn((inner,), seed=9)
    bias = randn((inner,), seed=10)
    assert_parity("LayerNormalization", [x, scale, bias], [(shape, F)], {"axis": axis, "epsilon": 1e-6})
    mean_shape = shape[:ax] + (1,) * (len(shape) - ax)
    assert_parity("LayerNormalization", [x, np.array([1.5], F)], [(shape, F), (mean_shape, F), (mean_shape, F)],
                  {"axis": axis})
    assert_parity("LayerNormalization", [x, np.array([0.75], F), np.array([-0.25], F)], [(shape, F)],
                  {"axis": axis})
    # Per-element Scale with no B, and with a scalar B (the kernels read an
    # absent or scalar operand through a zero step).
    assert_parity("LayerNormalization", [x, scale], [(shape, F)], {"axis": axis, "epsilon": 1e-6})
    assert_parity("LayerNormalization", [x, scale, np.array([-0.25], F)], [(shape, F)], {"axis": axis})
    assert outer > 0


def test_instancenorm(gpu):
    x = randn((2, 3, 17, 19), seed=11)
    assert_parity("InstanceNormalization", [x, randn((3,), seed=12), randn((3,), seed=13)], [(x.shape, F)],
                  {"epsilon": 1e-3})
    x2 = randn((1, 4, 640 * 64), seed=14)
    assert_parity("InstanceNormalization", [x2, randn((4,), seed=15), randn((4,), seed=16)], [(x2.shape, F)])


# One case per kernel path: a wave per plane (spatial <= 256, <= 1024; plane
# counts that leave the last block part-filled), a block per plane (<= 4096,
# <= 8192), and the split-plane path (whole and ragged 4096-element chunks).
@pytest.mark.parametrize("shape", [(3, 5, 7, 9), (2, 3, 17, 19), (2, 3, 40, 50), (1, 6, 80, 90), (1, 4, 40960),
                                   (2, 3, 100, 123), (1, 2, 3, 1)])
@pytest.mark.parametrize("offset", [0.0, 300.0])
def test_instancenorm_paths(gpu, shape, offset):
    x = (randn(shape, seed=31) + np.float32(offset)).astype(F)
    c = shape[1]
    assert_parity("InstanceNormalization", [x, randn((c,), seed=32), randn((c,), seed=33)], [(shape, F)],
                  {"epsilon": 1e-5})


@pytest.mark.parametrize("shape,axis,keepdims,last", [
    ((1024, 1024), 1, 1, 0), ((1024, 1024), 1, 0, 1), ((4, 5, 6), 1, 1, 0), ((4, 5, 6), 0, 0, 1), ((7,), 0, 0, 0),
])
def test_argmax(gpu, shape, axis, keepdims, last):
    x = rng(17).integers(-5, 5, shape).astype(F)  # many ties
    out = list(shape)
    if keepdims:
        out[axis] = 1
    else:
        out.pop(axis)
    attrs = {"axis": axis, "keepdims": keepdims, "select_last_index": last}
    assert_parity("ArgMax", [x], [(tuple(out), I)], attrs)
    assert_parity("ArgMax", [x.astype(I)], [(tuple(out), I)], attrs)


def test_argmax_nan(gpu):
    x = np.array([[np.nan, 5, 1], [1, np.nan, 3], [2, 2, np.nan], [np.nan, np.nan, np.nan]], F)
    for last in (0, 1):
        assert_parity("ArgMax", [x], [((4, 1), I)], {"axis": 1, "select_last_index": last})
    big = randn((3, 5000), seed=18)
    big[1, 0] = np.nan
    big[2, 100] = np.nan
    assert_parity("ArgMax", [big], [((3,), I)], {"axis": 1, "keepdims": 0})


@pytest.mark.parametrize("exclusive,reverse", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_cumsum(gpu, exclusive, reverse):
    x = randn((3, 7, 5), seed=19)
    for axis in (0, 1, -1):
        assert_parity("CumSum", [x, np.array(axis, I)], [(x.shape, F)], {"exclusive": exclusive, "reverse": reverse})
    xi = rng(20).integers(-9, 9, (4, 6)).astype(I)
    assert_parity("CumSum", [xi, np.array([1], I)], [(xi.shape, I)], {"exclusive": exclusive, "reverse": reverse})
    # Contiguous scan axes take the block scan per row: one chunk, several
    # chunks with a ragged last one, and int64 rows (exact).
    for shape in ((5, 300), (3, 2500)):
        xr = randn(shape, seed=21)
        assert_parity("CumSum", [xr, np.array(-1, I)], [(shape, F)], {"exclusive": exclusive, "reverse": reverse})
    xl = rng(22).integers(-2**40, 2**40, (2, 3000)).astype(I)
    assert_parity("CumSum", [xl, np.array(1, I)], [(xl.shape, I)], {"exclusive": exclusive, "reverse": reverse})
