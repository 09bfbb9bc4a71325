"""GPU parity: Resize, GridSample, Einsum and ConvTranspose against the
reference CpuDevice rows.

Resize nearest is a copy and must be bit-exact; linear Resize and
GridSample follow the reference's double-precision coordinate and weight
arithmetic step for step, so they are held to the same float32 bar as the
other float rows (|d| <= 1e-4 + 1e-4 |ref|). ConvTranspose runs as an MFMA
GEMM plus a tap gather in float32 (groups of 8+ input channels) or as a
direct kernel summing in double, where the reference scatters in float32
(same bar for both). Einsum equations that are batched matrix products run on
the GEMM engine, the rest on a double-sum walk (same bar)."""

import numpy as np
import pytest

from rowcheck import assert_parity, assert_same_error, randn, rng

pytestmark = pytest.mark.gpu

F, I = np.float32, np.int64
EXACT = {"rtol": 0.0, "atol": 0.0}
NONE = None


def _resize_scales(shape, scales):
    return tuple(int(np.floor(np.float64(d) * np.float64(np.float32(s)))) for d, s in zip(shape, scales))


TRANSFORMS = ["half_pixel", "pytorch_half_pixel", "align_corners", "asymmetric"]


@pytest.mark.parametrize("transform", TRANSFORMS)
@pytest.mark.parametrize("nearest", ["round_prefer_floor", "round_prefer_ceil", "floor", "ceil"])
def test_resize_nearest(gpu, transform, nearest):
    x = randn((2, 3, 7, 9), seed=1)
    attrs = {"mode": "nearest", "coordinate_transformation_mode": transform, "nearest_mode": nearest}
    for scales in ([1, 1, 2, 2], [1, 1, 0.6, 1.7], [1, 1, 3.3, 0.5]):
        out = _resize_scales(x.shape, scales)
        assert_parity("Resize", [x, NONE, np.array(scales, F)], [(out, F)], attrs, **EXACT)
    sizes = np.array([2, 3, 5, 13], I)
    assert_parity("Resize", [x, NONE, NONE, sizes], [(tuple(sizes), F)], attrs, **EXACT)
    # last output axis a multiple of 4: the four-outputs-per-thread kernel
    for sizes in ([2, 3, 5, 12], [2, 3, 11, 4], [1, 3, 7, 20]):
        assert_parity("Resize", [x, NONE, NONE, np.array(sizes, I)], [(tuple(sizes), F)], attrs, **EXACT)
    xi = rng(2).integers(-100, 100, (2, 3, 4, 5)).astype(I)
    assert_parity("Resize", [xi, NONE, np.array([1, 1, 2.5, 1.5], F)], [((2, 3, 10, 7), I)], attrs, **EXACT)


def test_resize_detector_upsample(gpu):
    """The detector's x2 nearest upsampling of a [8, 256, 20, 20] map (bit-exact)."""
    x = randn((8, 256, 20, 20), seed=3)
    assert_parity("Resize", [x, np.zeros((0,), F), np.array([1, 1, 2, 2], F)], [((8, 256, 40, 40), F)],
                  {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "floor"},
                  **EXACT)


@pytest.mark.parametrize("transform", TRANSFORMS)
def test_resize_linear(gpu, transform):
    x = randn((2, 3, 6, 8), seed=4)
    attrs = {"mode": "linear", "coordinate_transformation_mode": transform}
    for scales in ([1, 1, 2, 2], [1, 1, 0.5, 1.3], [1.5, 1, 1.7, 0.9]):
        out = _resize_scales(x.shape, scales)
        assert_parity("Resize", [x, NONE, np.array(scales, F)], [(out, F)], attrs)
    assert_parity("Resize", [x, NONE, NONE, np.array([2, 3, 11, 5], I)], [((2, 3, 11, 5), F)], attrs)
    x3 = randn((5, 6, 7), seed=5)  # three interpolating axes: eight taps
    assert_parity("Resize", [x3, NONE, np.array([1.5, 1.5, 1.5], F)], [((7, 9, 10), F)], attrs)


def test_resize_errors(gpu):
    x = randn((1, 1, 4, 4))
    s = np.array([1, 1, 2, 2], F)
    assert_same_error("Resize", [x, NONE, s], [((1, 1, 8, 8), F)], {"mode": "cubic"})
    assert_same_error("Resize", [x, NONE, s], [((1, 1, 8, 8), F)], {"coordinate_transformation_mode": "tf"})
    assert_same_error("Resize", [x, NONE, s], [((1, 1, 8, 8), F)], {"nearest_mode": "up"})
    assert_same_error("Resize", [x, NONE, s], [((1, 1, 8, 9), F)])
    assert_same_error("Resize", [x, NONE, s, np.array([1, 1, 8, 8], I)], [((1, 1, 8, 8), F)])
    assert_same_error("Resize", [x.astype(I), NONE, s], [((1, 1, 8, 8), I)], {"mode": "linear"})
    assert_same_error("Resize", [x, NONE, np.array([1, 1, 0.1, 2], F)], [((1, 1, 0, 8), F)])


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("padding", ["zeros", "border", "reflection"])
@pytest.mark.parametrize("align", [0, 1])
def test_grid_sample(gpu, mode, padding, align):
    x = randn((2, 3, 9, 11), seed=6)
    grid = (randn((2, 5, 7, 2), seed=7) * 0.8).astype(F)  # includes samples outside [-1, 1]
    grid[0, 0, 0] = [1.0, -1.0]
    grid[1, 4, 6] = [0.0, 0.0]
    grid[1, 3, 2] = [2.7, -3.9]
    attrs = {"mode": mode, "padding_mode": padding, "align_corners": align}
    assert_parity("GridSample", [x, grid], [((2, 3, 5, 7), F)], attrs)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("padding", ["zeros", "border", "reflection"])
@pytest.mark.parametrize("shape", [(1, 6, 33, 40, 21, 50), (3, 9, 16, 16, 40, 8), (2, 1, 5, 5, 3, 3)])
def test_grid_sample_channel_groups(gpu, mode, padding, shape):
    """Channel counts that do not fill the last group of four, and
    non-finite grid points (their taps fall outside the input)."""
    n, c, h, w, ho, wo = shape
    x = randn((n, c, h, w), seed=8)
    grid = (randn((n, ho, wo, 2), seed=9) * 0.9).astype(F)
    grid[0, 0, 0] = [np.inf, 0.5]
    grid[-1, -1, -1] = [-0.25, -np.inf]
    attrs = {"mode": mode, "padding_mode": padding, "align_corners": 0}
    assert_parity("GridSample", [x, grid], [((n, c, ho, wo), F)], attrs)


def test_grid_sample_errors(gpu):
    x = randn((1, 2, 4, 4))
    g = np.zeros((1, 3, 3, 2), F)
    assert_same_error("GridSample", [x, g], [((1, 2, 3, 3), F)], {"mode": "bicubic"})
    assert_same_error("GridSample", [x, g], [((1, 2, 3, 3), F)], {"padding_mode": "wrap"})
    assert_same_error("GridSample", [x, g], [((1, 2, 3, 3), F)], {"align_corners": 2})
    assert_same_error("GridSample", [x, g], [((1, 2, 3, 4), F)])
    assert_same_error("GridSample", [x, np.zeros((2, 3, 3, 2), F)], [((1, 2, 3, 3), F)])


EINSUM_CASES = [
    ("ij,jk->ik", [(5, 7), (7, 3)]),
    ("bij,bjk->bik", [(4, 5, 6), (4, 6, 3)]),
    ("bhqd,bhkd->bhqk", [(2, 3, 5, 8), (2, 3, 6, 8)]),
    ("ij,ij->", [(4, 5), (4, 5)]),
    ("i,j->ij", [(4,), (6,)]),
    ("ii->i", [(5, 5)]),
    ("ii", [(6, 6)]),
    ("ij->ji", [(3, 4)]),
    ("ijk->", [(3, 4, 5)]),
    ("ij,jk", [(3, 4), (4, 5)]),            # implicit output: ik
    ("Ab,bC->CA", [(3, 4), (4, 2)]),        # upper-case labels sort first
    ("...ij,...jk->...ik", [(2, 3, 4, 5), (3, 5, 6)]),
    ("...ij,jk->...ik", [(7, 3, 4), (4, 2)]),
    ("b...i,b...i->b...", [(2, 3, 4, 5), (2, 1, 4, 5)]),
    (" i j , j k -> i k ", [(2, 3), (3, 4)]),
]


@pytest.mark.parametrize("equation,shapes", EINSUM_CASES)
def test_einsum(gpu, equation, shapes):
    xs = [randn(s, seed=10 + i) for i, s in enumerate(shapes)]
    eq = equation.replace(" ", "")
    if "->" not in eq:
        counts = {}
        for c in eq.replace(",", ""):
            counts[c] = counts.get(c, 0) + 1
        eq = eq + "->" + "".join(sorted(c for c, n in counts.items() if n == 1))
    want = np.einsum(eq, *[x.astype(np.float64) for x in xs])
    assert_parity("Einsum", xs, [(want.shape, F)], {"equation": equation})


# (equation, shapes, lowered onto the GEMM engine). Contracted extents of 64
# and more make the fp32 MFMA sums differ from the double sums of the exact
# path in some bits, which is how the routing is observed.
EINSUM_ROUTES = [
    ("ij,jk->ik", [(96, 200), (200, 80)], True),
    ("ij,jk->ki", [(64, 128), (128, 96)], True),             # columns first: operands swap
    ("bij,bjk->bik", [(6, 64, 96), (6, 96, 48)], True),
    ("bhqd,bhkd->bhqk", [(2, 4, 64, 64), (2, 4, 80, 64)], True),
    ("bqhd,bkhd->bhqk", [(2, 64, 4, 32), (2, 48, 4, 32)], True),  # two batch groups, strided rows
    ("ijk,jkl->il", [(32, 16, 8), (16, 8, 40)], True),       # two contracted labels merge
    ("bi,bij->bj", [(8, 128), (8, 128, 64)], True),          # no row labels
    ("...ij,jk->...ik", [(7, 30, 64), (64, 20)], True),       # ellipsis rows merge
    ("ijk,kjl->il", [(16, 12, 10), (10, 12, 20)], False),    # contracted labels do not merge
    ("ij,kl->ikjl", [(8, 9), (10, 11)], False),              # rows and columns interleave
    ("ij,jk->i", [(32, 64), (64, 16)], False),               # k summed in one operand only
    ("ij->ji", [(30, 40)], False),                           # one operand
]


@pytest.mark.parametrize("equation,shapes,lowered", EINSUM_ROUTES)
def test_einsum_gemm_lowering(gpu, equation, shapes, lowered, monkeypatch):
    xs = [randn(s, seed=20 + i) for i, s in enumerate(shapes)]
    want = np.einsum(equation, *[x.astype(np.float64) for x in xs])
    got = assert_parity("Einsum", xs, [(want.shape, F)], {"equation": equation})[0]
    monkeypatch.setenv("NERT_HIP_EINSUM_EXACT", "1")
    exact = assert_parity("Einsum", xs, [(want.shape, F)], {"equation": equation})[0]
    assert np.array_equal(got, exact) != lowered, "lowered" if lowered else "exact path expected"


def test_einsum_errors(gpu):
    a, b = randn((3, 4)), randn((4, 5))
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ij,jk->iq"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ij,jk->ii"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ij,kk->ik"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ij,jk,kl->il"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "i1,jk->ik"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "...ij,jk"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ij..,jk->ik"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {"equation": "ijk,jk->ik"})
    assert_same_error("Einsum", [a, b], [((3, 6), F)], {"equation": "ij,jk->ik"})
    assert_same_error("Einsum", [a, b], [((3, 5), F)], {})
    c3 = randn((2, 3, 4))
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,jk"})           # implicit + ellipsis
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "abcd...,jk->...k"})   # rank below labels
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,j->...i"})      # no ellipsis, rank off
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "....ij,jk->...ik"})   # four dots
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,jk->...i.k"})   # dots in output
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,jk->...i1"})    # foreign output char
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,jk->...ii"})    # repeated output label
    assert_same_error("Einsum", [c3, b], [((3, 5), F)], {"equation": "...ij,jk->...iq"})    # unknown output label
    assert_same_error("Einsum", [c3], [((3, 5), F)], {"equation": "...ij,jk->...ik"})       # operand count (dots)
    assert_same_error("Einsum", [c3, randn((3, 4, 5))], [((2, 3, 5), F)],
                      {"equation": "...ij,...jk->...ik"})                                   # slots 2 vs 3
    wide = "".join(chr(c) for c in range(ord("a"), ord("z") + 1)) + "".join(
        chr(c) for c in range(ord("A"), ord("Y") + 1))                                      # 51 letters used
    assert_same_error("Einsum", [randn((1,) * 53)], [((1,), F)],
                      {"equation": wide + "...->" + "..."})                                 # no fresh labels left


def _einsum_outcome(equation, xs, out_shape):
    from rowcheck import run_hip, run_ref

    specs = [(out_shape, F)]
    want, ref_err = run_ref("Einsum", xs, specs, {"equation": equation}, name="fz")
    got, hip_err = run_hip("Einsum", xs, specs, {"equation": equation}, name="fz")
    if ref_err is not None or hip_err is not None:
        assert ref_err is not None and hip_err is not None, (equation, ref_err, hip_err)
        assert hip_err.message == ref_err.message, (equation, hip_err.message, ref_err.message)
        return False
    from rowcheck import compare

    compare(got[0], want[0], what=equation)
    return True


def test_einsum_random_equations(gpu):
    """Random equations, valid and not, over a small alphabet: the HIP row
    accepts exactly what the reference row accepts, rejects with the same
    message, and agrees with it on the result."""
    r = rng(77)
    letters = "ijkAB"
    accepted = 0
    for case in range(300):
        n_ops = int(r.integers(1, 3)) if case % 17 else int(r.integers(1, 4))
        subs, shapes = [], []
        extents = {c: int(r.integers(1, 4)) for c in letters}
        batch = [int(r.integers(1, 4)) for _ in range(3)]
        for _ in range(n_ops):
            labels = [letters[int(k)] for k in r.integers(0, len(letters), int(r.integers(0, 4)))]
            dims = [extents[c] for c in labels]
            if r.random() < 0.4:
                nb = int(r.integers(0, 3))
                pos = int(r.integers(0, len(labels) + 1))
                bd = [1 if r.random() < 0.3 else b for b in batch[3 - nb:]]
                labels = labels[:pos] + ["..."] + labels[pos:]
                dims = dims[:pos] + bd + dims[pos:]
            if r.random() < 0.08 and dims:
                dims[int(r.integers(0, len(dims)))] += 1          # size clash
            if r.random() < 0.05:
                labels.append(r.choice(["1", ".", "..", "_"]))     # syntax error
            subs.append("".join(labels))
            shapes.append(tuple(dims))
        eq = ",".join(subs)
        if r.random() < 0.85:
            out = sorted({c for s in subs for c in s if c.isalpha()})
            out = list(r.permutation(out))[: int(r.integers(0, len(out) + 1))]
            if any("..." in s for s in subs) and r.random() < 0.8:
                out.insert(int(r.integers(0, len(out) + 1)), "...")
            if r.random() < 0.05:
                out.append(r.choice(["q", "i", "."]))
            eq += "->" + "".join(out)
        xs = [randn(s, seed=case * 7 + i) if len(s) else np.array(randn((1,), seed=case)[0], F) for i, s in
              enumerate(shapes)]
        try:
            out_shape = np.einsum(eq, *[x.astype(np.float64) for x in xs]).shape
        except Exception:  # numpy rejects it too: any output shape, errors are compared
            out_shape = (1,)
        accepted += _einsum_outcome(eq, xs, out_shape)
    assert accepted > 100, f"only {accepted} of 300 random equations were accepted"


@pytest.mark.parametrize("geom", [
    dict(x=(2, 4, 5, 6), w=(4, 3, 3, 3), attrs={}),
    dict(x=(2, 4, 5, 6), w=(4, 3, 3, 3), attrs={"strides": [2, 2]}),
    dict(x=(1, 6, 7, 5), w=(6, 2, 4, 3), attrs={"strides": [3, 2], "pads": [1, 0, 2, 1], "group": 3}),
    dict(x=(1, 4, 5, 5), w=(4, 4, 3, 3), attrs={"strides": [2, 2], "dilations": [2, 1], "output_padding": [1, 1]}),
    dict(x=(2, 8, 16, 16), w=(8, 4, 2, 2), attrs={"strides": [2, 2]}),          # 2x learned upsampling
    dict(x=(1, 3, 4, 4), w=(3, 2, 3, 3), attrs={"pads": [1, 1, 1, 1], "auto_pad": "VALID"}),
])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv_transpose(gpu, geom, with_bias):
    inputs, spec, a = _conv_transpose_case(geom, with_bias)
    assert_parity("ConvTranspose", inputs, spec, a)


def _conv_transpose_case(geom, with_bias):
    a = geom["attrs"]
    x, w = randn(geom["x"], seed=20), randn(geom["w"], seed=21)
    s, d = a.get("strides", [1, 1]), a.get("dilations", [1, 1])
    op, p = a.get("output_padding", [0, 0]), a.get("pads", [0, 0, 0, 0])
    if a.get("auto_pad") == "VALID":
        p = [0, 0, 0, 0]
    m = w.shape[1] * a.get("group", 1)
    oh = s[0] * (x.shape[2] - 1) + op[0] + d[0] * (w.shape[2] - 1) + 1 - p[0] - p[2]
    ow = s[1] * (x.shape[3] - 1) + op[1] + d[1] * (w.shape[3] - 1) + 1 - p[1] - p[3]
    inputs = [x, w] + ([randn((m,), seed=22)] if with_bias else [])
    return inputs, [((x.shape[0], m, oh, ow), F)], a


# Groups of 8 or more input channels run as an MFMA GEMM plus a tap gather;
# (geometry, lowered). The exact path (NERT_HIP_CONVT_EXACT=1) sums in double,
# so with 64 channels per group the two differ in some bits.
CONVT_GEMM_GEOMS = [
    (dict(x=(2, 16, 9, 11), w=(16, 8, 3, 3), attrs={"strides": [2, 2], "pads": [1, 1, 1, 1]}), True),
    (dict(x=(1, 32, 8, 8), w=(32, 6, 4, 4), attrs={"strides": [2, 2], "pads": [1, 1, 1, 1], "group": 2}), True),
    (dict(x=(2, 8, 7, 6), w=(8, 5, 3, 3), attrs={"dilations": [2, 2]}), True),
    (dict(x=(1, 12, 5, 5), w=(12, 4, 3, 3), attrs={"strides": [3, 2], "pads": [1, 0, 2, 1],
                                                   "output_padding": [2, 1], "dilations": [1, 2]}), True),
    (dict(x=(4, 64, 16, 16), w=(64, 32, 4, 4), attrs={"strides": [2, 2], "pads": [1, 1, 1, 1]}), True),
    (dict(x=(2, 4, 5, 6), w=(4, 3, 3, 3), attrs={"strides": [2, 2]}), False),
]


@pytest.mark.parametrize("geom,lowered", CONVT_GEMM_GEOMS)
def test_conv_transpose_gemm_path(gpu, geom, lowered, monkeypatch):
    inputs, spec, a = _conv_transpose_case(geom, True)
    got = assert_parity("ConvTranspose", inputs, spec, a)[0]
    monkeypatch.setenv("NERT_HIP_CONVT_EXACT", "1")
    exact = assert_parity("ConvTranspose", inputs, spec, a)[0]
    if lowered and geom["x"][1] // geom["attrs"].get("group", 1) >= 64:
        assert not np.array_equal(got, exact), "expected the GEMM path"
    if not lowered:
        assert np.array_equal(got, exact), "expected the direct path"


def test_conv_transpose_errors(gpu):
    x, w = randn((1, 4, 3, 3)), randn((4, 2, 3, 3))
    assert_same_error("ConvTranspose", [x, w], [((1, 2, 5, 6), F)])
    assert_same_error("ConvTranspose", [x, randn((3, 2, 3, 3))], [((1, 2, 5, 5), F)])
    assert_same_error("ConvTranspose", [x, w, randn((3,))], [((1, 2, 5, 5), F)])
    assert_same_error("ConvTranspose", [x, w], [((1, 2, 5, 5), F)], {"strides": [1, 1, 1]})
