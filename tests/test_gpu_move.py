"""GPU parity: movement rows (Transpose, Concat, Split, Slice, Expand, Tile,
Squeeze, Unsqueeze, Pad) against the reference CpuDevice rows. All outputs
are copies, so every comparison is bit-exact, float32 included."""

import numpy as np
import pytest

from rowcheck import assert_parity, assert_same_error, randn, rng

pytestmark = pytest.mark.gpu

F, I, B = np.float32, np.int64, np.bool_
EXACT = {"rtol": 0.0, "atol": 0.0}


def _data(shape, dtype, seed=0):
    if dtype == F:
        return randn(shape, seed=seed)
    if dtype == I:
        return rng(seed).integers(-1 << 40, 1 << 40, shape).astype(I)
    return rng(seed).integers(0, 2, shape).astype(B)


@pytest.mark.parametrize("shape,perm", [
    ((16, 197, 12, 64), [0, 2, 1, 3]),   # ViT head split
    ((16, 12, 197, 64), [0, 2, 1, 3]),   # ViT head merge
    ((16, 12, 197, 64), [0, 1, 3, 2]),   # K^T: batched LDS-tile transpose
    ((8, 84, 8400), [0, 2, 1]),          # detector head, ragged tiles
    ((3, 37, 45), [0, 2, 1]),
    ((5, 33, 7, 40), [3, 1, 0, 2]),
    ((9, 40, 3), [1, 0, 2]),             # 3-element runs: scalar path
    ((2048, 1024), [1, 0]),
    ((2, 3, 4, 5, 6), [4, 2, 0, 3, 1]),
    ((3, 1, 5), [1, 2, 0]),
    ((7,), [0]),
    ((4, 5, 6), None),                    # default: reversed axes
])
@pytest.mark.parametrize("dtype", [F, I, B])
def test_transpose(gpu, shape, perm, dtype):
    x = _data(shape, dtype, seed=len(shape))
    p = perm if perm is not None else list(range(len(shape)))[::-1]
    out = tuple(shape[i] for i in p)
    attrs = {} if perm is None else {"perm": perm}
    assert_parity("Transpose", [x], [(out, dtype)], attrs, **EXACT)


def test_transpose_errors(gpu):
    x = randn((2, 3, 4))
    assert_same_error("Transpose", [x], [((3, 2, 4), F)], {"perm": [1, 0]})
    assert_same_error("Transpose", [x], [((3, 2, 4), F)], {"perm": [1, 1, 2]})
    assert_same_error("Transpose", [x], [((2, 3, 4), F)], {"perm": [1, 0, 2]})
    assert_same_error("Transpose", [x], [((3, 2, 4), I)], {"perm": [1, 0, 2]})
    assert_parity("Transpose", [np.zeros((0, 3), F)], [((3, 0), F)], {"perm": [1, 0]})


@pytest.mark.parametrize("shapes,axis", [
    ([(16, 1, 768), (16, 196, 768)], 1),  # ViT class token
    ([(2, 3, 4), (2, 5, 4), (2, 1, 4)], 1),
    ([(2, 3), (4, 3)], 0),
    ([(2, 3), (2, 7)], -1),
    ([(5,), (0,), (3,)], 0),
    ([(1, 2, 3, 4)], 3),
    ([(8, 64, 20, 20), (8, 128, 20, 20), (8, 32, 20, 20)], 1),  # detector neck: 16-byte units
    ([(70000, 1), (70000, 2)], 1),                              # more rows than one grid column
    ([(3, i + 1) for i in range(9)], 1),                        # nine inputs: one copy per input
])
@pytest.mark.parametrize("dtype", [F, I, B])
def test_concat(gpu, shapes, axis, dtype):
    xs = [_data(s, dtype, seed=i) for i, s in enumerate(shapes)]
    out = np.concatenate(xs, axis=axis).shape
    assert_parity("Concat", xs, [(out, dtype)], {"axis": axis}, **EXACT)


def test_concat_errors(gpu):
    a, b = randn((2, 3)), randn((2, 4))
    assert_same_error("Concat", [a, b], [((4, 3), F)], {"axis": 0})
    assert_same_error("Concat", [a, b], [((2, 7), F)], {"axis": 2})
    assert_same_error("Concat", [a, b.astype(I)], [((2, 7), F)], {"axis": 1})
    assert_same_error("Concat", [a, randn((2, 3, 1))], [((2, 7), F)], {"axis": 1})
    assert_same_error("Concat", [a, b], [((2, 8), F)], {"axis": 1})
    assert_parity("Concat", [a, b], [((2, 7), F)], **EXACT)  # default axis 1


@pytest.mark.parametrize("dtype", [F, I])
def test_split(gpu, dtype):
    x = _data((6, 10, 4), dtype, seed=3)
    assert_parity("Split", [x], [((6, 5, 4), dtype)] * 2, {"axis": 1}, **EXACT)
    assert_parity("Split", [x, np.array([2, 3, 5], I)], [((6, 2, 4), dtype), ((6, 3, 4), dtype), ((6, 5, 4), dtype)],
                  {"axis": -2}, **EXACT)
    assert_parity("Split", [x, np.array([0, 6], I)], [((0, 10, 4), dtype), ((6, 10, 4), dtype)], **EXACT)
    # schema < 13: sizes as an attribute
    assert_parity("Split", [x], [((6, 10, 1), dtype), ((6, 10, 3), dtype)], {"axis": 2, "split": [1, 3]},
                  schema_version=11, **EXACT)
    # schema 18: num_outputs with a shorter last chunk
    assert_parity("Split", [x], [((6, 4, 4), dtype), ((6, 4, 4), dtype), ((6, 2, 4), dtype)],
                  {"axis": 1, "num_outputs": 3}, schema_version=18, **EXACT)


def test_split_errors(gpu):
    x = randn((6, 10))
    assert_same_error("Split", [x], [((6, 3), F)] * 3, {"axis": 1})
    assert_same_error("Split", [x, np.array([4, 4], I)], [((6, 4), F)] * 2, {"axis": 1})
    assert_same_error("Split", [x, np.array([4, 6], I)], [((6, 4), F), ((6, 5), F)], {"axis": 1})
    assert_same_error("Split", [x], [((6, 5), F)] * 2, {"axis": 2})
    assert_same_error("Split", [x.astype(B)], [((6, 5), B)] * 2, {"axis": 1})
    assert_same_error("Split", [x], [((6, 4), F), ((6, 4), F), ((6, 2), F)], {"axis": 1, "num_outputs": 3},
                      schema_version=13)


def _slice_shape(shape, starts, ends, axes, steps):
    idx = [slice(None)] * len(shape)
    for s, e, a, st in zip(starts, ends, axes, steps):
        idx[a] = slice(s, e, st)
    return np.empty(shape)[tuple(idx)].shape


@pytest.mark.parametrize("starts,ends,axes,steps", [
    ([1], [3], None, None),
    ([0, 1], [2, 100], [0, 2], None),
    ([-1], [-1000], [1], [-1]),
    ([5, 0], [1, -1], [2, 0], [-2, 2]),
    ([2], [2], [1], [1]),          # empty selection
    ([100], [200], [0], [1]),      # clamped empty
    ([-3, 1], [100, 5], [-1, -2], [3, 1]),
])
@pytest.mark.parametrize("dtype", [F, I, B])
def test_slice(gpu, starts, ends, axes, steps, dtype):
    x = _data((4, 6, 8), dtype, seed=5)
    ax = axes if axes is not None else list(range(len(starts)))
    st = steps if steps is not None else [1] * len(starts)
    out = _slice_shape(x.shape, starts, ends, [a % 3 for a in ax], st)
    inputs = [x, np.array(starts, I), np.array(ends, I)]
    if axes is not None or steps is not None:
        inputs.append(np.array(ax, I))
    if steps is not None:
        inputs.append(np.array(st, I))
    assert_parity("Slice", inputs, [(out, dtype)], **EXACT)


def test_slice_vit_token(gpu):
    # class-token pick in ViT heads: [:, 0:1, :] of (16, 197, 768)
    x = randn((16, 197, 768), seed=6)
    assert_parity("Slice", [x, np.array([0], I), np.array([1], I), np.array([1], I)], [((16, 1, 768), F)], **EXACT)


def test_slice_errors(gpu):
    x = randn((4, 6))
    assert_same_error("Slice", [x, np.array([0], I), np.array([2, 3], I)], [((2, 6), F)])
    assert_same_error("Slice", [x, np.array([0], I), np.array([2], I), np.array([0], I), np.array([0], I)],
                      [((2, 6), F)])
    assert_same_error("Slice", [x, np.array([0], I), np.array([2], I), np.array([2], I)], [((2, 6), F)])
    assert_same_error("Slice", [x, np.array([0], I), np.array([2], I)], [((3, 6), F)])
    assert_same_error("Slice", [x, np.array([0.0], F), np.array([2], I)], [((2, 6), F)])


@pytest.mark.parametrize("shape,target", [
    ((3, 1), [3, 4]), ((1,), [2, 3, 5]), ((2, 1, 4), [3, 2, 5, 4]), ((4,), [1]), ((1, 1), [6, 1, 7]),
    ((1, 768), [16 * 197, 768]),
])
@pytest.mark.parametrize("dtype", [F, I, B])
def test_expand(gpu, shape, target, dtype):
    x = _data(shape, dtype, seed=7)
    out = np.broadcast_shapes(shape, tuple(target))
    assert_parity("Expand", [x, np.array(target, I)], [(out, dtype)], **EXACT)


def test_expand_errors(gpu):
    x = randn((3, 2))
    assert_same_error("Expand", [x, np.array([3, 4], I)], [((3, 4), F)])
    assert_same_error("Expand", [x, np.array([0, 2], I)], [((0, 2), F)])
    assert_same_error("Expand", [x, np.array([3, 2], I)], [((3, 3), F)])


@pytest.mark.parametrize("shape,reps", [((2, 3), [2, 2]), ((4,), [5]), ((1, 3, 2), [3, 1, 4]), ((2, 5, 3), [1, 1, 1])])
@pytest.mark.parametrize("dtype", [F, I, B])
def test_tile(gpu, shape, reps, dtype):
    x = _data(shape, dtype, seed=8)
    out = tuple(d * r for d, r in zip(shape, reps))
    assert_parity("Tile", [x, np.array(reps, I)], [(out, dtype)], **EXACT)


def test_tile_errors(gpu):
    x = randn((2, 3))
    assert_same_error("Tile", [x, np.array([2], I)], [((4, 3), F)])
    assert_same_error("Tile", [x, np.array([2, 0], I)], [((4, 0), F)])
    assert_same_error("Tile", [x, np.array([2, 2], I)], [((4, 5), F)])


def test_squeeze_unsqueeze(gpu):
    for dtype in (F, I, B):
        x = _data((3, 1, 4, 1), dtype, seed=9)
        assert_parity("Squeeze", [x, np.array([1, 3], I)], [((3, 4), dtype)], **EXACT)
        assert_parity("Squeeze", [x], [((3, 4), dtype)], **EXACT)
        y = _data((3, 4), dtype, seed=10)
        assert_parity("Unsqueeze", [y, np.array([0, -1], I)], [((1, 3, 4, 1), dtype)], **EXACT)
        assert_parity("Unsqueeze", [y], [((3, 1, 4), dtype)], {"axes": [1]}, schema_version=11, **EXACT)
    x = randn((3, 4))
    assert_same_error("Squeeze", [x], [((3, 5), F)])
    assert_same_error("Unsqueeze", [x, np.array([0, 0], I)], [((1, 1, 3, 4), F)])
    assert_same_error("Unsqueeze", [x, np.array([5], I)], [((3, 4, 1), F)])
    assert_same_error("Unsqueeze", [x, np.array([0], I)], [((3, 4, 1), F)])
    assert_same_error("Unsqueeze", [x], [((1, 3, 4), F)], {"axes": [0]}, schema_version=13)


@pytest.mark.parametrize("mode", ["constant", "reflect", "edge"])
@pytest.mark.parametrize("dtype", [F, I])
def test_pad(gpu, mode, dtype):
    x = _data((2, 3, 5, 6), dtype, seed=11)
    pads = [0, 0, 2, 3, 0, 1, 4, 5]
    out = (2, 4, 11, 14)
    attrs = {"mode": mode}
    assert_parity("Pad", [x, np.array(pads, I)], [(out, dtype)], attrs, **EXACT)
    value = np.array(2.5, F) if dtype == F else np.array(-7, I)
    assert_parity("Pad", [x, np.array(pads, I), value], [(out, dtype)], attrs, **EXACT)
    # axes input: pad only the last two axes; negative pads crop
    assert_parity("Pad", [x, np.array([1, -1, 2, 3], I), None, np.array([-2, -1], I)], [((2, 3, 8, 8), dtype)],
                  attrs, **EXACT)
    # reflect beyond one period
    if mode != "constant":
        y = _data((3, 4), dtype, seed=12)
        assert_parity("Pad", [y, np.array([5, 9, 6, 11], I)], [((14, 24), dtype)], attrs, **EXACT)


def test_pad_errors(gpu):
    x = randn((3, 4))
    assert_same_error("Pad", [x, np.array([1, 1, 1], I)], [((5, 6), F)])
    assert_same_error("Pad", [x, np.array([1, 1, 1, 1], I)], [((5, 7), F)])
    assert_same_error("Pad", [x, np.array([1, 1], I), None, np.array([0, 0], I)], [((4, 4), F)])
    assert_same_error("Pad", [x, np.array([1, 1, 1, 1], I)], [((5, 6), F)], {"mode": "wrap"})
    assert_same_error("Pad", [x, np.array([1, 1, 1, 1], I), np.array(1, I)], [((5, 6), F)])
