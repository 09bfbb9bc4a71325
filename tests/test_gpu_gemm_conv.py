"""GPU parity: Gemm, MatMul and Conv rows against the reference CpuDevice and
the numpy restatement, from the reference's own known-answer cases up to the
BASELINE.json configs at full size."""

import numpy as np
import pytest

from nert_amd.device import DeviceArray, run_node
from oracle import restate
from rowcheck import assert_parity, assert_same_error, compare, randn, uniform

pytestmark = pytest.mark.gpu

F = np.float32


def _hip(op, inputs, out_shape, attrs=None):
    dev_in = [None if x is None else DeviceArray.from_host(x) for x in inputs]
    out = DeviceArray(out_shape, F)
    run_node(op, dev_in, [out], attrs)
    return out.to_host()


# --- known answers from test/hip_kernels_test.cpp -------------------------

def test_gemm_small_exact(gpu):
    a = np.array([[1, 2, 3], [4, 5, 6]], F)
    b = np.array([[7, 8], [9, 10], [11, 12]], F)
    got = assert_parity("Gemm", [a, b], [((2, 2), F)], name="gemm0")
    assert np.array_equal(got[0], np.array([[58, 64], [139, 154]], F))  # hip_kernels_test.cpp:97-98


def test_gemm_transposed_with_bias(gpu):
    a = np.array([1, 2, 3, 4, 5, 6], F).reshape(3, 2)
    b = np.array([1, 0, 0, 1, 2, 1, 0, 2, 1, 1, 0, 1], F).reshape(4, 3)
    c = np.array([0.5, -0.5, 1.0, 2.0], F)
    attrs = {"transA": 1, "transB": 1, "alpha": 2.0, "beta": 0.5}
    assert_parity("Gemm", [a, b, c], [((2, 4), F)], attrs, name="gemm1")


def test_gemm_rejects_mismatch(gpu):
    msg = assert_same_error("Gemm", [np.ones((2, 3), F), np.ones((2, 2), F)], [((2, 2), F)], name="gemm_bad")
    assert "contraction dimension mismatch" in msg


def test_matmul_batched_broadcast(gpu):
    a = np.array([1, 2, 3, 4, 5, 6], F).reshape(2, 3)
    b = np.array([1, 0, 0, 1, 1, 1, 2, 0, 0, 2, 1, 0], F).reshape(2, 3, 2)
    got = assert_parity("MatMul", [a, b], [((2, 2, 2), F)], name="mm0")
    assert np.array_equal(got[0].ravel(), np.array([4, 5, 10, 11, 5, 4, 14, 10], F))


def test_matmul_promoted_vector(gpu):
    a = np.array([1, 2, 3], F)
    b = np.array([[1, 2], [3, 4], [5, 6]], F)
    got = assert_parity("MatMul", [a, b], [((2,), F)], name="mm1")
    assert np.array_equal(got[0], np.array([22, 28], F))


def test_conv_pointwise_no_bias(gpu):
    x = np.arange(1, 9, dtype=F).reshape(1, 2, 2, 2)
    w = np.array([1, 0, 0, 1, 1, 1], F).reshape(3, 2, 1, 1)
    got = assert_parity("Conv", [x, w], [((1, 3, 2, 2), F)], name="cv0")
    assert np.array_equal(got[0].ravel(), np.array([1, 2, 3, 4, 5, 6, 7, 8, 6, 8, 10, 12], F))


def test_conv_padded_3x3_with_bias(gpu):
    x = np.arange(1, 10, dtype=F).reshape(1, 1, 3, 3)
    w = np.ones((1, 1, 3, 3), F)
    b = np.array([10], F)
    got = assert_parity("Conv", [x, w, b], [((1, 1, 3, 3), F)], {"pads": [1, 1, 1, 1]}, name="cv1")
    assert np.array_equal(got[0].ravel(), np.array([22, 31, 26, 37, 55, 43, 34, 49, 38], F))


def test_conv_depthwise_with_bias(gpu):
    x = np.arange(1, 9, dtype=F).reshape(1, 2, 2, 2)
    w = np.array([2, 3], F).reshape(2, 1, 1, 1)
    b = np.array([1, -1], F)
    got = assert_parity("Conv", [x, w, b], [((1, 2, 2, 2), F)], {"group": 2}, name="cv2")
    assert np.array_equal(got[0].ravel(), np.array([3, 5, 7, 9, 14, 17, 20, 23], F))


def test_conv_same_upper_asymmetric(gpu):
    x = ((np.arange(18) % 13) - 6).astype(F).reshape(1, 2, 3, 3) * F(0.5)
    w = ((np.arange(16) % 7) - 3).astype(F).reshape(2, 2, 2, 2) * F(0.25)
    b = np.array([1.5, -2.5], F)
    assert_parity("Conv", [x, w, b], [((1, 2, 3, 3), F)], {"auto_pad": "SAME_UPPER"}, name="cv_same")


# --- randomized parity against the reference rows -------------------------

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 13, 5), (33, 65, 17), (130, 97, 301), (256, 128, 64)])
def test_gemm_trans_random(gpu, ta, tb, m, n, k):
    a = uniform((k, m) if ta else (m, k), seed=m)
    b = uniform((n, k) if tb else (k, n), seed=n + 1)
    c = uniform((n,), seed=k + 2)
    assert_parity("Gemm", [a, b, c], [((m, n), F)], {"transA": ta, "transB": tb, "alpha": 0.75, "beta": -1.25})


def test_gemm_rank2_bias_and_no_bias(gpu):
    a = uniform((40, 70), seed=1)
    b = uniform((70, 90), seed=2)
    c = uniform((40, 90), seed=3)
    assert_parity("Gemm", [a, b, c], [((40, 90), F)])
    assert_parity("Gemm", [a, b], [((40, 90), F)], {"alpha": 3.0})


@pytest.mark.parametrize("ashape,bshape,oshape", [
    ((3, 4, 5), (5, 6), (3, 4, 6)),
    ((2, 1, 4, 5), (3, 5, 7), (2, 3, 4, 7)),
    ((5,), (2, 5, 3), (2, 3)),
    ((2, 3, 4), (4,), (2, 3)),
    ((4,), (4,), ()),
    ((2, 12, 33, 16), (2, 12, 16, 33), (2, 12, 33, 33)),
    ((1, 9, 130, 70), (70, 64), (1, 9, 130, 64)),
])
def test_matmul_shapes(gpu, ashape, bshape, oshape):
    a = uniform(ashape, seed=len(ashape))
    b = uniform(bshape, seed=len(bshape) + 7)
    assert_parity("MatMul", [a, b], [(oshape, F)])


CONV_CASES = [
    # x shape, w shape, attrs
    ((2, 3, 17, 19), (8, 3, 3, 3), {"pads": [1, 1, 1, 1]}),
    ((1, 4, 15, 15), (6, 4, 5, 3), {"strides": [2, 1], "pads": [2, 1, 2, 1]}),
    ((2, 6, 12, 12), (6, 2, 3, 3), {"group": 3, "dilations": [2, 2], "pads": [2, 2, 2, 2]}),
    ((1, 3, 32, 32), (16, 3, 7, 7), {"strides": [2, 2], "pads": [3, 3, 3, 3]}),
    ((2, 16, 14, 14), (32, 16, 1, 1), {"strides": [2, 2]}),
    ((1, 4, 9, 9), (5, 4, 2, 2), {"auto_pad": "SAME_LOWER", "strides": [2, 2]}),
    ((1, 4, 9, 9), (5, 4, 3, 3), {"auto_pad": "VALID"}),
    ((2, 3, 20), (4, 3, 5), {"pads": [2, 2]}),                   # 1-D
    ((1, 2, 5, 6, 7), (3, 2, 2, 3, 3), {"pads": [1, 0, 1, 1, 1, 1]}),  # 3-D
    ((1, 8, 10, 10), (8, 1, 3, 3), {"group": 8, "pads": [1, 1, 1, 1]}),  # depthwise
    ((4, 64, 14, 14), (128, 64, 3, 3), {"pads": [1, 1, 1, 1], "strides": [2, 2]}),
    # windows that tile the input exactly run as a GEMM over patch columns
    ((2, 3, 32, 32), (48, 3, 16, 16), {"strides": [16, 16]}),    # the ViT patch embedding, small
    ((3, 5, 12, 20), (7, 5, 2, 4), {"strides": [2, 4]}),        # non-square windows, odd channels
    ((1, 4, 9, 9), (6, 4, 3, 3), {"strides": [3, 3]}),          # KW not a multiple of 4: the gather kernel
]


@pytest.mark.parametrize("xs,ws,attrs", CONV_CASES)
def test_conv_random(gpu, xs, ws, attrs):
    x = randn(xs, seed=sum(xs))
    w = randn(ws, seed=sum(ws), scale=0.2)
    b = randn((ws[0],), seed=3, scale=0.1)
    ref = restate.conv(x, w, b, attrs.get("strides"), attrs.get("dilations"), attrs.get("pads"),
                       attrs.get("group", 1), attrs.get("auto_pad", "NOTSET"))
    got = assert_parity("Conv", [x, w, b], [(ref.shape, F)], attrs)
    compare(got[0], ref, what="conv vs restatement")


# 3x3 convolutions with C_g a multiple of 8 take the LDS-patch kernel; these
# cover tiles that straddle images, several images per tile, strides 2 and 3,
# dilation, asymmetric pads, groups, deep split-K and a too-wide patch that
# falls back to the tap-major kernel.
HALO_CASES = [
    ((2, 64, 56, 56), (64, 64, 3, 3), {"pads": [1, 1, 1, 1]}),
    ((5, 64, 7, 7), (128, 64, 3, 3), {"pads": [1, 1, 1, 1]}),
    ((3, 32, 29, 31), (48, 32, 3, 3), {"pads": [1, 1, 1, 1], "strides": [2, 2]}),
    ((2, 16, 20, 18), (40, 16, 3, 3), {"pads": [2, 2, 2, 2], "dilations": [2, 2]}),
    ((2, 8, 15, 13), (24, 8, 3, 3), {"pads": [0, 1, 2, 0]}),
    ((2, 8, 11, 12), (8, 8, 3, 3), {}),
    ((2, 32, 12, 12), (48, 16, 3, 3), {"pads": [1, 1, 1, 1], "group": 2}),
    ((2, 256, 9, 9), (96, 256, 3, 3), {"pads": [1, 1, 1, 1]}),
    ((1, 8, 20, 20), (8, 8, 3, 3), {"strides": [3, 3], "pads": [1, 1, 1, 1]}),
    ((2, 16, 10, 9), (16, 16, 3, 3), {"strides": [1, 2], "dilations": [2, 1], "pads": [2, 0, 1, 1]}),
    ((1, 8, 6, 700), (16, 8, 3, 3), {"pads": [1, 1, 1, 1]}),
]


@pytest.mark.parametrize("xs,ws,attrs", HALO_CASES)
def test_conv_lds_patch(gpu, xs, ws, attrs):
    x = randn(xs, seed=sum(xs) + 1)
    w = randn(ws, seed=sum(ws) + 1, scale=float(np.sqrt(2.0 / (ws[1] * 9))))
    b = randn((ws[0],), seed=5, scale=0.1)
    ref = restate.conv(x, w, b, attrs.get("strides"), attrs.get("dilations"), attrs.get("pads"),
                       attrs.get("group", 1), "NOTSET")
    got = assert_parity("Conv", [x, w, b], [(ref.shape, F)], attrs)
    compare(got[0], ref, what="conv vs restatement")


def test_conv_lds_patch_repeatable(gpu):
    """The first call of a geometry picks its tile configuration by timing;
    later calls reuse it, so repeated calls are bit-identical."""
    x = randn((3, 32, 20, 20), seed=70)
    w = randn((64, 32, 3, 3), seed=71, scale=0.1)
    b = randn((64,), seed=72)
    first = _hip("Conv", [x, w, b], (3, 64, 20, 20), {"pads": [1, 1, 1, 1]})
    for _ in range(2):
        assert np.array_equal(_hip("Conv", [x, w, b], (3, 64, 20, 20), {"pads": [1, 1, 1, 1]}), first)


# --- BASELINE.json configs at full size -----------------------------------

def test_vit_patch_embedding_full_size(gpu):
    """configs[3]'s patch embedding at full size: [16,3,224,224] * [768,3,16,16]
    at stride 16, as patch columns and one batched GEMM, against the
    restatement."""
    xs, ws, attrs = (16, 3, 224, 224), (768, 3, 16, 16), {"strides": [16, 16]}
    x, w, b = randn(xs, seed=70), randn(ws, seed=71, scale=0.02), randn((768,), seed=72, scale=0.02)
    got = _hip("Conv", [x, w, b], _conv_out(xs, ws, attrs), attrs)
    compare(got, restate.conv(x, w, b, [16, 16], None, None, 1, "NOTSET"), what="ViT patch embedding")


def test_config0_conv_3x3(gpu):
    """X[1,64,56,56], W[64,64,3,3], B[64], pad 1 -> [1,64,56,56]."""
    x = randn((1, 64, 56, 56), seed=0)
    w = randn((64, 64, 3, 3), seed=1, scale=np.sqrt(2 / 576))
    b = randn((64,), seed=2, scale=0.01)
    assert_parity("Conv", [x, w, b], [((1, 64, 56, 56), F)], {"pads": [1, 1, 1, 1]})


def test_config1a_batched_matmul(gpu):
    """configs[1](a): [8,1024,1024] x [8,1024,1024] against the restatement."""
    a = uniform((8, 1024, 1024), seed=10)
    b = uniform((8, 1024, 1024), seed=11)
    got = _hip("MatMul", [a, b], (8, 1024, 1024))
    compare(got, restate.matmul(a, b), what="cfg1a")


def test_config1b_gemm_transb(gpu):
    """configs[1](b): A[2048,4096] x B[1024,4096]^T + C[1024]."""
    a = uniform((2048, 4096), seed=12)
    b = uniform((1024, 4096), seed=13)
    c = uniform((1024,), seed=14)
    got = _hip("Gemm", [a, b, c], (2048, 1024), {"transB": 1, "alpha": 1.0, "beta": 1.0})
    compare(got, restate.gemm(a, b, c, trans_b=1), what="cfg1b")


@pytest.mark.parametrize("m,n,k", [(7, 45, 72), (32, 33, 8), (1, 1000, 512), (20, 300, 4096)])
def test_skinny_gemm_shapes(gpu, m, n, k):
    """Few rows with K contiguous in both operands (transB): the skinny kernel's
    territory, with ragged M and N, short and long K, a 2-D C and alpha/beta."""
    a = uniform((m, k), seed=m + 1)
    b = uniform((n, k), seed=n + 2)
    assert_parity("Gemm", [a, b, uniform((n,), seed=3)], [((m, n), F)], {"transB": 1})
    assert_parity("Gemm", [a, b, uniform((m, n), seed=4)], [((m, n), F)],
                  {"transB": 1, "alpha": 0.5, "beta": -2.0})


def test_config1c_skinny_gemm(gpu):
    """configs[1](c): A[32,512] x B[1000,512]^T + bias, against the reference row."""
    a = uniform((32, 512), seed=15)
    b = uniform((1000, 512), seed=16)
    c = uniform((1000,), seed=17)
    assert_parity("Gemm", [a, b, c], [((32, 1000), F)], {"transB": 1})


# --- FusedConv: the runner's Conv -> Add -> Relu fusion ------------------------

FUSED_CASES = [
    ((2, 64, 14, 14), (64, 64, 3, 3), {"pads": [1, 1, 1, 1]}),                      # tap-major, split-K
    ((1, 256, 7, 7), (512, 256, 3, 3), {"pads": [1, 1, 1, 1]}),                     # deep split-K
    ((2, 3, 32, 32), (16, 3, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),     # stem kernel (C=3)
    ((24, 3, 224, 224), (64, 3, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),  # stem, 2-3 blocks per workgroup
    ((2, 32, 9, 9), (48, 32, 1, 1), {}),                                            # pointwise shape
    ((1, 64, 20, 20), (64, 16, 3, 3), {"pads": [1, 1, 1, 1], "group": 4}),          # groups
    ((2, 3, 64, 64), (40, 3, 8, 8), {"strides": [8, 8]}),                           # patch columns + GEMM
]


@pytest.mark.parametrize("xs,ws,attrs", FUSED_CASES)
@pytest.mark.parametrize("with_z", [False, True])
def test_fused_conv_bit_identical(gpu, xs, ws, attrs, with_z):
    """FusedConv == Conv row, then float32 Add, then Relu, bit for bit; and
    within the Conv tolerance of the reference rows."""
    x, w, b = randn(xs, seed=40), randn(ws, seed=41, scale=0.1), randn((ws[0],), seed=42)
    conv = _hip("Conv", [x, w, b], _conv_out(xs, ws, attrs), attrs)
    z = randn(conv.shape, seed=43) if with_z else None
    want = conv + z if with_z else conv
    want = np.where(want > 0, want, np.float32(0)).astype(F)
    fattrs = dict(attrs, activation="Relu")
    got = _hip("FusedConv", [x, w, b] + ([z] if with_z else []), conv.shape, fattrs)
    assert np.array_equal(got, want)
    # without an activation and without a bias
    got = _hip("FusedConv", [x, w, None] + ([z] if with_z else []), conv.shape, attrs)
    plain = _hip("Conv", [x, w], conv.shape, attrs)
    assert np.array_equal(got, plain + z if with_z else plain)
    ref_conv = restate.conv(x, w, b, **_restate_args(attrs))
    ref = ref_conv + z if with_z else ref_conv
    compare(_hip("FusedConv", [x, w, b] + ([z] if with_z else []), conv.shape, fattrs),
            np.maximum(ref, 0).astype(F), what="FusedConv vs reference")


@pytest.mark.parametrize("xs,ws,attrs", FUSED_CASES + [
    ((2, 16, 40, 40), (32, 16, 3, 3), {"pads": [1, 1, 1, 1], "strides": [2, 2]}),  # detector stage
])
@pytest.mark.parametrize("with_z", [False, True])
def test_fused_conv_silu_bit_identical(gpu, xs, ws, attrs, with_z):
    """FusedConv(activation="Silu") == Conv row, [Add], Sigmoid row, Mul row,
    bit for bit; and within the Conv tolerance of the reference rows."""
    x, w, b = randn(xs, seed=44, scale=2.0), randn(ws, seed=45, scale=0.1), randn((ws[0],), seed=46)
    out = _conv_out(xs, ws, attrs)
    t = _hip("Conv", [x, w, b], out, attrs)
    z = randn(t.shape, seed=47) if with_z else None
    if with_z:
        t = _hip("Add", [t, z], out)
    want = _hip("Mul", [t, _hip("Sigmoid", [t], out)], out)
    got = _hip("FusedConv", [x, w, b] + ([z] if with_z else []), out, dict(attrs, activation="Silu"))
    assert np.array_equal(got, want)
    r = restate.conv(x, w, b, **_restate_args(attrs)).astype(np.float64)
    if with_z:
        r = r + z
    compare(got, (r / (1.0 + np.exp(-r))).astype(F), what="FusedConv Silu vs reference")


@pytest.mark.parametrize("ashape,n,alpha,bias,gelu", [
    ((2, 197, 64), 96, None, True, False),     # projection + bias
    ((2, 197, 64), 96, None, True, True),      # fc1 + bias + Gelu
    ((3, 4, 33, 16), 33, 0.125, False, False), # scaled attention scores
    ((5, 40), 24, 2.0, True, True),
])
def test_fused_matmul_bit_identical(gpu, ashape, n, alpha, bias, gelu):
    """FusedMatMul == MatMul, Mul(alpha), Add(bias), Div/Erf/Add/Mul/Mul rows."""
    a = randn(ashape, seed=60)
    w = randn((ashape[-1], n), seed=61, scale=0.2)
    b = randn((n,), seed=62)
    out = ashape[:-1] + (n,)
    y = _hip("MatMul", [a, w], out)
    if alpha is not None:
        y = _hip("Mul", [y, np.array(alpha, F)], out)
    if bias:
        y = _hip("Add", [y, b], out)
    attrs = {}
    if alpha is not None:
        attrs["alpha"] = alpha
    if gelu:
        c1, c2, c3 = np.float32(np.sqrt(2.0)), np.float32(1.0), np.float32(0.5)
        e = _hip("Erf", [_hip("Div", [y, np.array(c1, F)], out)], out)
        e = _hip("Add", [e, np.array(c2, F)], out)
        y = _hip("Mul", [_hip("Mul", [y, e], out), np.array(c3, F)], out)
        attrs.update({"activation": "Gelu", "gelu_div": float(c1), "gelu_add": float(c2), "gelu_mul": float(c3)})
    got = _hip("FusedMatMul", [a, w] + ([b] if bias else []), out, attrs)
    assert np.array_equal(got, y)


def test_fused_matmul_errors(gpu):
    from nert_amd.device import NertError

    a, w = randn((4, 8)), randn((8, 6))
    with pytest.raises(NertError, match=r"FusedMatMul \(node 'n'\): unsupported activation 'Tanh'"):
        _hip("FusedMatMul", [a, w], (4, 6), {"activation": "Tanh"})
    with pytest.raises(NertError, match=r"FusedMatMul \(node 'n'\): bias must be float32 \[N\]"):
        _hip("FusedMatMul", [a, w, randn((5,))], (4, 6))
    with pytest.raises(NertError, match=r"FusedMatMul \(node 'n'\): output shape does not match the operands"):
        _hip("FusedMatMul", [a, w], (4, 7))


def test_fused_conv_errors(gpu):
    from nert_amd.device import NertError

    x, w = randn((1, 4, 5, 5)), randn((4, 4, 3, 3))
    with pytest.raises(NertError, match=r"FusedConv \(node 'n'\): unsupported activation 'Tanh'"):
        _hip("FusedConv", [x, w], (1, 4, 3, 3), {"activation": "Tanh"})
    with pytest.raises(NertError, match=r"FusedConv \(node 'n'\): the summed input must be float32"):
        _hip("FusedConv", [x, w, None, randn((1, 4, 3, 2))], (1, 4, 3, 3))
    with pytest.raises(NertError, match=r"FusedConv \(node 'n'\): output shape does not match the convolution"):
        _hip("FusedConv", [x, w], (1, 4, 5, 5))


def _conv_out(xs, ws, attrs):
    pads = attrs.get("pads", [0, 0, 0, 0])
    s = attrs.get("strides", [1, 1])
    d = attrs.get("dilations", [1, 1])
    oh = (xs[2] + pads[0] + pads[2] - (d[0] * (ws[2] - 1) + 1)) // s[0] + 1
    ow = (xs[3] + pads[1] + pads[3] - (d[1] * (ws[3] - 1) + 1)) // s[1] + 1
    return (xs[0], ws[0], oh, ow)


def _restate_args(attrs):
    return {"strides": attrs.get("strides"), "pads": attrs.get("pads"), "group": attrs.get("group", 1)}


# --- small-channel convolutions (image stems) --------------------------------

@pytest.mark.parametrize("xs,ws,attrs", [
    ((4, 3, 64, 64), (64, 3, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),     # ResNet stem
    ((2, 3, 70, 50), (16, 3, 3, 3), {"pads": [1, 1, 1, 1], "strides": [2, 2]}),     # detector stem, ragged
    ((2, 1, 33, 31), (100, 1, 5, 4), {"pads": [2, 1, 2, 2], "dilations": [2, 1]}),  # M > 64, even KW
    ((2, 4, 20, 20), (8, 2, 3, 3), {"pads": [1, 1, 1, 1], "group": 2}),             # groups
    ((3, 3, 45, 61), (100, 3, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),    # 7x7, two channel blocks
    ((1, 2, 30, 30), (64, 2, 7, 7), {"pads": [2, 3, 1, 3], "dilations": [1, 2]}),   # 7x7, C=2, dilated
    ((2, 3, 40, 40), (24, 3, 3, 5), {"pads": [2, 2, 2, 2], "strides": [1, 2], "dilations": [2, 1]}),  # 5 taps
    ((1, 4, 36, 36), (32, 4, 4, 8), {"pads": [1, 3, 2, 4], "strides": [2, 2]}),     # 8 taps, C=4
    # 7 taps: filter rows taken in pairs (an even count, an odd count, dilated rows)
    ((2, 2, 40, 40), (32, 2, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),     # 14 rows
    ((2, 1, 33, 35), (40, 1, 5, 7), {"pads": [2, 3, 2, 3], "strides": [2, 2]}),     # 5 rows
    ((1, 4, 30, 44), (48, 4, 3, 7), {"pads": [1, 3, 1, 3], "strides": [2, 2], "dilations": [2, 1]}),  # 12 rows
    # 1029 pixel blocks on 512 workgroups: the last 5 blocks run as quarter blocks
    ((21, 3, 224, 224), (64, 3, 7, 7), {"pads": [3, 3, 3, 3], "strides": [2, 2]}),
])
def test_small_channel_conv(gpu, xs, ws, attrs):
    x, w, b = randn(xs, seed=50), randn(ws, seed=51), randn((ws[0],), seed=52)
    assert_parity("Conv", [x, w, b], [(_conv_out(xs, ws, attrs), F)], attrs)
    assert_parity("Conv", [x, w], [(_conv_out(xs, ws, attrs), F)], attrs)  # no bias


@pytest.mark.parametrize("xs,ws,attrs", [
    ((2, 3, 70, 50), (16, 3, 3, 3), {"pads": [1, 1, 1, 1], "strides": [2, 2]}),     # detector stem, ragged
    ((2, 4, 20, 20), (8, 2, 3, 3), {"pads": [1, 1, 1, 1], "group": 2}),             # groups
    ((2, 2, 17, 19), (32, 2, 4, 4), {"pads": [1, 2, 2, 1], "strides": [1, 2]}),     # K = 32, M = 32
    ((1, 1, 9, 9), (5, 1, 3, 3), {"pads": [2, 2, 2, 2], "dilations": [2, 2]}),      # dilated, C = 1
])
@pytest.mark.parametrize("cand", [300, 301])
def test_small_channel_conv_candidates(gpu, tmp_path, xs, ws, attrs, cand):
    """Both small-channel candidates -- the MFMA patch kernel (300) and the
    direct VALU kernel for tiny filters and channel counts (301) -- forced:
    Conv within tolerance of the restatement, the fused epilogue equal to
    Conv + Add + Relu bit for bit."""
    x, w, b = randn(xs, seed=60), randn(ws, seed=61, scale=0.2), randn((ws[0],), seed=62)
    z = randn(_conv_out(xs, ws, attrs), seed=63)
    paths = {k: str(tmp_path / f"{k}.npy") for k in ("x", "w", "b", "z", "out1", "out2")}
    for k, v in (("x", x), ("w", w), ("b", b), ("z", z)):
        np.save(paths[k], v)
    _run_forced(cand, paths, attrs, tune=False)
    conv = np.load(paths["out1"])
    compare(conv, restate.conv(x, w, b, attrs.get("strides"), attrs.get("dilations"), attrs.get("pads"),
                               attrs.get("group", 1), "NOTSET"), what=f"candidate {cand}")
    want = conv + z
    assert np.array_equal(np.load(paths["out2"]), np.where(want > 0, want, np.float32(0)).astype(F))


def test_small_channel_conv_nonfinite_inputs(gpu):
    """A padded (zero-weight) tap must not turn an inf input into NaN."""
    x = randn((1, 3, 40, 40), seed=53)
    x[0, 1, 10, 13] = np.inf
    x[0, 2, 30, 7] = -np.inf
    w, b = randn((64, 3, 7, 7), seed=54), randn((64,), seed=55)
    attrs = {"pads": [3, 3, 3, 3], "strides": [2, 2]}
    assert_parity("Conv", [x, w, b], [(_conv_out(x.shape, w.shape, attrs), F)], attrs)


# --- every 3x3 configuration, forced ----------------------------------------

_FORCED = r"""
import json, sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd.device import DeviceArray, run_node
x = np.load({x!r}); w = np.load({w!r}); b = np.load({b!r}); z = np.load({z!r})
def hip(op, ins, shape, attrs):
    dev = [DeviceArray.from_host(a) for a in ins]
    out = DeviceArray(shape, np.float32)
    run_node(op, dev, [out], attrs)
    return out.to_host()
a = json.loads({attrs!r})
y = hip("Conv", [x, w, b], z.shape, a)
np.save({out1!r}, y)
np.save({out2!r}, hip("FusedConv", [x, w, b, z], z.shape, dict(a, activation="Relu")))
# a third launch of the same geometry: split tiles finished in the kernel
# leave their counters at zero for the next launch
assert np.array_equal(hip("Conv", [x, w, b], z.shape, a), y), "second Conv launch differs"
"""


@pytest.mark.parametrize("batch,hw", [(17, 32), (32, 28)])
@pytest.mark.parametrize("cand", [0, 9, 14, 18, 19, 22, 23] + list(range(24, 33)))
def test_conv_lds_patch_forced_configs(gpu, tmp_path, batch, hw, cand):
    """Each 3x3 configuration (tile shapes with 8- and 16-channel K steps,
    split counts, and the tail split that cuts the last partial round of tiles
    along the channels: 16 tiles in 8 pieces, or 136 tiles in halves)
    computes the same convolution: forced in
    a child process, compared with the restatement and with the fused
    epilogue applied by hand."""
    x = randn((batch, 64, hw, hw), seed=80)
    w = randn((64, 64, 3, 3), seed=81, scale=0.06)
    b = randn((64,), seed=82, scale=0.1)
    z = randn((batch, 64, hw, hw), seed=83)
    paths = {k: str(tmp_path / f"{k}.npy") for k in ("x", "w", "b", "z", "out1", "out2")}
    for k, v in (("x", x), ("w", w), ("b", b), ("z", z)):
        np.save(paths[k], v)
    _run_forced(cand, paths, {"pads": [1, 1, 1, 1]})
    conv = np.load(paths["out1"])
    ref = restate.conv(x, w, b, None, None, [1, 1, 1, 1], 1, "NOTSET")
    compare(conv, ref, what=f"candidate {cand}")
    want = conv + z
    assert np.array_equal(np.load(paths["out2"]), np.where(want > 0, want, np.float32(0)).astype(F))


_PAIR = """
import json, sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd.device import DeviceArray, run_node
x, w, b, z, w2, b2 = (np.load(p) for p in {ins!r})
a = dict(json.loads({attrs!r}), activation="Relu")
dev = lambda v: DeviceArray.from_host(v)
def pair(zz, bb2):
    y, y2 = DeviceArray(z.shape, np.float32), DeviceArray(z.shape, np.float32)
    run_node("FusedConv", [dev(x), dev(w), dev(b), None if zz is None else dev(zz), dev(w2),
                           None if bb2 is None else dev(bb2)], [y, y2], a)
    return y.to_host(), y2.to_host()
y, y2 = pair(None, b2)
single = DeviceArray(z.shape, np.float32)
run_node("FusedConv", [dev(x), dev(w), dev(b)], [single], a)
yz, y2z = pair(z, None)
single_z = DeviceArray(z.shape, np.float32)
run_node("FusedConv", [dev(x), dev(w), dev(b), dev(z)], [single_z], a)
again = pair(None, b2)
np.savez({out!r}, y=y, y2=y2, single=single.to_host(), yz=yz, y2z=y2z, single_z=single_z.to_host(),
         again_y=again[0], again_y2=again[1])
"""


@pytest.mark.parametrize("xs,m", [((2, 64, 56, 56), 128), ((2, 128, 28, 28), 256), ((2, 256, 14, 14), 512),
                                  ((3, 32, 15, 13), 32), ((2, 64, 16, 16), 64)])
@pytest.mark.parametrize("cand", [None, 1, 5, 9, 13, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 27, 28, 30, 31])
def test_conv_pair_matches_separate_rows(gpu, tmp_path, xs, m, cand):
    """A 3x3 pad-1 conv paired with the 1x1 shortcut conv of its input at the
    same stride (six-input FusedConv, one launch of the halo kernel): the 3x3
    output equals the single FusedConv row bit for bit under the same forced
    configuration (None: the tuned choice, then only within the tolerance),
    the 1x1 output matches the restatement of the 1x1 conv with and without
    its bias, the summand path is applied to the 3x3 output only, and a
    second launch is bit-identical (split counters reset)."""
    import json
    import os
    import subprocess
    import sys

    stride = 1 if xs[2] == 16 else 2
    attrs = {"pads": [1, 1, 1, 1], "strides": [stride, stride]}
    x = randn(xs, seed=130)
    w = randn((m, xs[1], 3, 3), seed=131, scale=0.05)
    b = randn((m,), seed=132, scale=0.1)
    w2 = randn((m, xs[1], 1, 1), seed=133, scale=0.1)
    b2 = randn((m,), seed=134, scale=0.1)
    z = randn(_conv_out(xs, w.shape, attrs), seed=135)
    ins = []
    for k, v in (("x", x), ("w", w), ("b", b), ("z", z), ("w2", w2), ("b2", b2)):
        ins.append(str(tmp_path / f"{k}.npy"))
        np.save(ins[-1], v)
    out = str(tmp_path / "out.npz")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    if cand is not None:
        # A candidate that does not fit the geometry falls back to the fixed
        # default (not a table or timed choice, which the paired family makes
        # apart from the single conv).
        env["NERT_HIP_CONV_CANDIDATE"] = str(cand)
        env["NERT_HIP_CONV_TUNE"] = "0"
        env["NERT_HIP_TUNE_TABLE"] = os.devnull
    subprocess.run([sys.executable, "-c", _PAIR.format(root=root, ins=ins, attrs=json.dumps(attrs), out=out)],
                   env=env, check=True, timeout=120)
    r = np.load(out)
    conv = restate.conv(x, w, b, attrs["strides"], None, attrs["pads"], 1, "NOTSET")
    relu = lambda v: np.where(v > 0, v, np.float32(0)).astype(F)
    want2 = restate.conv(x, w2, b2, attrs["strides"], None, [0, 0, 0, 0], 1, "NOTSET")
    compare(r["y2"], want2, what=f"paired 1x1, candidate {cand}")
    compare(r["y2z"], restate.conv(x, w2, None, attrs["strides"], None, [0, 0, 0, 0], 1, "NOTSET"),
            what=f"paired 1x1 without bias, candidate {cand}")
    if cand is not None:
        assert np.array_equal(r["y"], r["single"]) and np.array_equal(r["yz"], r["single_z"])
    compare(r["y"], relu(conv), what=f"paired 3x3, candidate {cand}")
    compare(r["yz"], relu((conv.astype(np.float64) + z).astype(F)), rtol=2e-4, atol=2e-4,
            what=f"paired 3x3 with summand, candidate {cand}")
    assert np.array_equal(r["again_y"], r["y"]) and np.array_equal(r["again_y2"], r["y2"])


def test_conv_pair_rejects_bad_operands(gpu):
    """The paired FusedConv row checks the 1x1 operands before launching and
    names the node in its message."""
    from nert_amd.device import NertError

    x = DeviceArray.from_host(randn((1, 8, 8, 8), seed=1))
    w = DeviceArray.from_host(randn((16, 8, 3, 3), seed=2))
    w2 = DeviceArray.from_host(randn((16, 8, 1, 1), seed=4))
    y = DeviceArray((1, 16, 4, 4), F)
    y2 = DeviceArray((1, 16, 4, 4), F)
    attrs = {"pads": [1, 1, 1, 1], "strides": [2, 2]}
    cases = [
        ([x, w, None, None, DeviceArray.from_host(randn((16, 8, 3, 3), seed=3)), None], [y, y2], attrs,
         "the paired weight must be float32 [M, C, 1, 1]"),
        ([x, w, None, None, w2, None], [y, DeviceArray((1, 16, 3, 3), F)], attrs,
         "the paired output must be float32 with the first output's shape"),
        ([x, w, None, None, w2, DeviceArray.from_host(randn((8,), seed=5))], [y, y2], attrs,
         "the paired bias must be float32 [M]"),
        ([x, w, None, None, w2, None], [y, y2], dict(attrs, dilations=[2, 2], pads=[2, 2, 2, 2]),
         "a paired conv needs a 3x3 first conv with pad 1, dilation 1, group 1"),
    ]
    for ins, outs, a, msg in cases:
        with pytest.raises(NertError) as err:
            run_node("FusedConv", ins, outs, a, name="p")
        assert "FusedConv (node 'p'): " + msg in str(err.value), str(err.value)


@pytest.mark.parametrize("batch,hw", [(17, 32), (32, 28), (3, 9)])
@pytest.mark.parametrize("cand", [2, 3, 11, 15, 16, 17, 18, 19, 20, 21, 22, 23, 25, 26, 28, 29, 31, 32])
def test_conv_split_fixup_matches_reduce_kernels(gpu, tmp_path, batch, hw, cand):
    """Split-K and tail-split configurations finish their split tiles inside
    the conv kernel (the last workgroup of a tile to arrive adds the parts in
    part order); the result equals, bit for bit, the same configuration
    with the parts summed by the separate reduce kernels
    (NERT_HIP_SPLIT_FIXUP=0), for Conv and for the fused epilogue. Where a
    candidate does not fit the geometry, both runs take the fixed default
    (NERT_HIP_CONV_TUNE=0) rather than a timed choice."""
    x = randn((batch, 64, hw, hw), seed=84)
    w = randn((64, 64, 3, 3), seed=85, scale=0.06)
    b = randn((64,), seed=86, scale=0.1)
    z = randn((batch, 64, hw, hw), seed=87)
    outs = []
    for fixup in (True, False):
        paths = {k: str(tmp_path / f"{k}{int(fixup)}.npy") for k in ("x", "w", "b", "z", "out1", "out2")}
        for k, v in (("x", x), ("w", w), ("b", b), ("z", z)):
            np.save(paths[k], v)
        _run_forced(cand, paths, {"pads": [1, 1, 1, 1]}, fixup=fixup, tune=False)
        outs.append((np.load(paths["out1"]), np.load(paths["out2"])))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    compare(outs[0][0], restate.conv(x, w, b, None, None, [1, 1, 1, 1], 1, "NOTSET"), what=f"candidate {cand}")


@pytest.mark.parametrize("xs,ws,attrs", [
    ((2, 256, 14, 14), (512, 256, 1, 1), {"strides": [2, 2]}),                    # few tiles, long K
    ((1, 120, 20, 20), (32, 60, 3, 3), {"pads": [1, 1, 1, 1], "group": 2}),       # grouped gather, long K
])
@pytest.mark.parametrize("cand", [100, 101, 102, 104, 105, 106, 107])
def test_conv_gather_split_fixup_matches_reduce_kernels(gpu, tmp_path, xs, ws, attrs, cand):
    """The gather / tap-major conv kernels' split-K tiles, finished inside the
    kernel, equal the reduce-kernel sums bit for bit (Conv and the fused
    epilogue), and the restatement within tolerance."""
    x, w, b = randn(xs, seed=94), randn(ws, seed=95, scale=0.1), randn((ws[0],), seed=96)
    z = randn(_conv_out(xs, ws, attrs), seed=97)
    outs = []
    for fixup in (True, False):
        paths = {k: str(tmp_path / f"{k}{int(fixup)}.npy") for k in ("x", "w", "b", "z", "out1", "out2")}
        for k, v in (("x", x), ("w", w), ("b", b), ("z", z)):
            np.save(paths[k], v)
        _run_forced(cand, paths, attrs, fixup=fixup, tune=False)
        outs.append((np.load(paths["out1"]), np.load(paths["out2"])))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    compare(outs[0][0], restate.conv(x, w, b, attrs.get("strides"), None, attrs.get("pads"), attrs.get("group", 1),
                                     "NOTSET"), what=f"candidate {cand}")


def _run_forced(cand, paths, attrs, fixup=True, tune=True):
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, NERT_HIP_CONV_CANDIDATE=str(cand))
    if not fixup:
        env["NERT_HIP_SPLIT_FIXUP"] = "0"
    if not tune:
        env["NERT_HIP_CONV_TUNE"] = "0"
    subprocess.run([sys.executable, "-c", _FORCED.format(root=root, attrs=json.dumps(attrs), **paths)], env=env,
                   check=True, timeout=120)


@pytest.mark.parametrize("xs,ws,attrs", [
    ((4, 64, 56, 56), (128, 64, 1, 1), {"strides": [2, 2]}),   # ResNet downsampling
    ((2, 256, 14, 14), (512, 256, 1, 1), {"strides": [2, 2]}),
    ((3, 24, 9, 11), (40, 24, 1, 1), {"strides": [1, 2], "pads": [1, 0, 0, 1]}),
    ((2, 32, 8, 8), (48, 16, 1, 1), {"group": 2}),
])
@pytest.mark.parametrize("cand", [100, 101, 102, 103, 104, 105, 106, 107])
def test_conv_1x1_forced_configs(gpu, tmp_path, xs, ws, attrs, cand):
    """Every configuration of the other conv kernels, the direct 1x1 kernel
    (103), the small-tile shapes (104, 105) and the 32-deep K steps (106,
    107) included, forced: matches the
    restatement, and the fused epilogue matches Conv + Add + Relu bit for
    bit."""
    x, w, b = randn(xs, seed=90), randn(ws, seed=91, scale=0.1), randn((ws[0],), seed=92)
    out = _conv_out(xs, ws, attrs)
    z = randn(out, seed=93)
    paths = {k: str(tmp_path / f"{k}.npy") for k in ("x", "w", "b", "z", "out1", "out2")}
    for k, v in (("x", x), ("w", w), ("b", b), ("z", z)):
        np.save(paths[k], v)
    _run_forced(cand, paths, attrs)
    conv = np.load(paths["out1"])
    compare(conv, restate.conv(x, w, b, attrs.get("strides"), None, attrs.get("pads"), attrs.get("group", 1),
                               "NOTSET"), what=f"candidate {cand}")
    want = conv + z
    assert np.array_equal(np.load(paths["out2"]), np.where(want > 0, want, np.float32(0)).astype(F))


# --- every GEMM candidate, forced ------------------------------------------

GEMM_FORCED = [
    ("MatMul", [(24, 197, 64), (24, 64, 197)], {}),                 # attention scores (K = 64)
    ("MatMul", [(24, 197, 197), (24, 197, 64)], {}),                # attention x V (K = 197, unaligned rows)
    ("MatMul", [(3, 70, 33), (3, 33, 45)], {}),                     # ragged M, N, K
    ("MatMul", [(96, 200), (200, 80)], {}),                         # one batch
    ("Gemm", [(50, 37), (60, 37)], {"transB": 1}),                  # K contiguous in B
    ("Gemm", [(37, 50), (37, 60)], {"transA": 1}),                  # A transposed
    ("Gemm", [(40, 1100), (1100, 24)], {}),                         # two-level accumulation (K > 1024)
]


_GEMM_SPLIT = r"""
import sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd.device import DeviceArray, run_node
import os
cases = {cases!r}
outs = {{}}
for ci, (op, shapes, attrs, out) in enumerate(cases):
    xs = [np.random.default_rng(70 + ci * 4 + i).uniform(-1, 1, s).astype(np.float32) for i, s in enumerate(shapes)]
    for cand in {cands!r}:
        os.environ["NERT_HIP_GEMM_CANDIDATE"] = str(cand)
        dev = [DeviceArray.from_host(a) for a in xs]
        res = []
        for rep in range(2):
            y = DeviceArray(tuple(out), np.float32)
            run_node(op, dev, [y], attrs)
            res.append(y.to_host())
        assert np.array_equal(res[0], res[1]), (ci, cand, "second launch differs")
        outs[f"{{ci}}_{{cand}}"] = res[0]
np.savez({path!r}, **outs)
"""


def test_gemm_split_fixup_matches_reduce_kernels(gpu, tmp_path):
    """GEMM split-K tiles finished inside the kernel (parts summed in double
    by the tile's last workgroup, in split order) equal, bit for bit, the
    same configuration summed by the separate reduce kernels
    (NERT_HIP_SPLIT_FIXUP=0): every split candidate, forced, on shapes with a
    K remainder, a two-level K range and batches; two launches in a row."""
    import os
    import subprocess
    import sys

    cases = [("MatMul", [(3, 70, 333), (3, 333, 45)], {}, (3, 70, 45)),
             ("Gemm", [(40, 1100), (1100, 24)], {}, (40, 24)),
             ("Gemm", [(512, 512), (512, 512)], {"transB": 1}, (512, 512)),
             ("MatMul", [(96, 200), (200, 80)], {}, (96, 80))]
    cands = [i for i in range(25) if i != 12 and (i if i < 12 else i - 13) % 4 in (2, 3)]
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    got = []
    for fixup in (True, False):
        path = str(tmp_path / f"gemm{int(fixup)}.npz")
        env = dict(os.environ)
        if not fixup:
            env["NERT_HIP_SPLIT_FIXUP"] = "0"
        subprocess.run([sys.executable, "-c", _GEMM_SPLIT.format(root=root, cases=cases, cands=cands, path=path)],
                       env=env, check=True, timeout=120)
        got.append(np.load(path))
    assert sorted(got[0].files) == sorted(got[1].files)
    for k in got[0].files:
        assert np.array_equal(got[0][k], got[1][k]), k


@pytest.mark.parametrize("candidate", list(range(25)))
@pytest.mark.parametrize("op,shapes,attrs", GEMM_FORCED)
def test_gemm_every_candidate(gpu, monkeypatch, candidate, op, shapes, attrs):
    """Each tile shape x split count and the skinny kernel, forced with
    NERT_HIP_GEMM_CANDIDATE wherever it applies, against the reference row."""
    monkeypatch.setenv("NERT_HIP_GEMM_CANDIDATE", str(candidate))
    xs = [uniform(s, seed=50 + i) for i, s in enumerate(shapes)]
    if op == "MatMul":
        out = np.matmul(np.zeros(shapes[0], F), np.zeros(shapes[1], F)).shape
    else:
        m = shapes[0][1] if attrs.get("transA") else shapes[0][0]
        n = shapes[1][0] if attrs.get("transB") else shapes[1][1]
        out = (m, n)
    assert_parity(op, xs, [(out, F)], attrs)


@pytest.mark.parametrize("candidate", list(range(25)))
@pytest.mark.parametrize("xs,ws,strides", [
    ((3, 5, 16, 16), (6, 5, 4, 4), [4, 4]),    # K = 80: a checked K tail; 48 pixels: edge tiles
    ((2, 3, 64, 64), (40, 3, 16, 8), [16, 8]),  # non-square windows, 64 pixels
])
def test_patch_conv_every_gemm_candidate(gpu, monkeypatch, candidate, xs, ws, strides):
    """A convolution whose windows tile its input runs as one GEMM whose B
    loader reads the patches from X in place; under every GEMM candidate
    (tile shapes, split counts) forced with NERT_HIP_GEMM_CANDIDATE, against
    the reference row."""
    monkeypatch.setenv("NERT_HIP_GEMM_CANDIDATE", str(candidate))
    x, w, b = uniform(xs, seed=80), uniform(ws, seed=81), uniform((ws[0],), seed=82)
    attrs = {"strides": strides}
    assert_parity("Conv", [x, w, b], [(_conv_out(xs, ws, attrs), F)], attrs)


_PACKED = """
import json, os, sys
import numpy as np
sys.path.insert(0, {root!r})
from nert_amd.device import DeviceArray, run_node
x, w, b, w2, b2 = (np.load(p) for p in {ins!r})
a = json.loads({attrs!r})
m, cg = w.shape[:2]
wp = np.ascontiguousarray(w.reshape(m, cg // 8, 8, 9).transpose(0, 1, 3, 2)).reshape(w.shape)
dev = lambda v: DeviceArray.from_host(v)
shape = [x.shape[0], m] + [(x.shape[2 + i] + 2 - 3) // a["strides"][i] + 1 for i in range(2)]
out = {{}}
for cand in {cands!r}:
    os.environ["NERT_HIP_CONV_CANDIDATE"] = str(cand)
    for packed in (False, True):
        y = DeviceArray(shape, np.float32)
        ins = [dev(x), dev(w), dev(b)] + ([None, None, None, dev(wp)] if packed else [])
        run_node("FusedConv", ins, [y], a)
        out[f"single_{{cand}}_{{int(packed)}}"] = y.to_host()
        if a.get("group", 1) == 1:
            y, y2 = DeviceArray(shape, np.float32), DeviceArray(shape, np.float32)
            ins = [dev(x), dev(w), dev(b), None, dev(w2), dev(b2)] + ([dev(wp)] if packed else [])
            run_node("FusedConv", ins, [y, y2], a)
            out[f"pair_{{cand}}_{{int(packed)}}"] = y.to_host()
            out[f"pair2_{{cand}}_{{int(packed)}}"] = y2.to_host()
np.savez({out!r}, **out)
"""


@pytest.mark.parametrize("xs,m,stride,group", [((2, 64, 20, 20), 64, 1, 1), ((2, 32, 15, 13), 48, 2, 1),
                                              ((1, 16, 9, 9), 32, 1, 1), ((2, 32, 12, 12), 48, 1, 2)])
def test_conv_packed_weights_bit_identical(gpu, tmp_path, xs, m, stride, group):
    """FusedConv with W also given packed (seventh input, the 3x3 LDS-patch
    kernel's order) against the same row without it, single and (group 1)
    paired with a 1x1 shortcut, under every 3x3 configuration forced in turn
    (8- and 16-channel blocks, split and tail pieces, two groups; tuning
    off): bit-identical; the tuned result matches the restatement."""
    import json
    import os
    import subprocess
    import sys

    attrs = {"pads": [1, 1, 1, 1], "strides": [stride, stride], "activation": "Relu", "group": group}
    x = randn(xs, seed=140)
    w = randn((m, xs[1] // group, 3, 3), seed=141, scale=0.05)
    b = randn((m,), seed=142, scale=0.1)
    w2 = randn((m, xs[1], 1, 1), seed=143, scale=0.1)
    b2 = randn((m,), seed=144, scale=0.1)
    ins = []
    for k, v in (("x", x), ("w", w), ("b", b), ("w2", w2), ("b2", b2)):
        ins.append(str(tmp_path / f"{k}.npy"))
        np.save(ins[-1], v)
    out = str(tmp_path / "out.npz")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, NERT_HIP_CONV_TUNE="0", NERT_HIP_TUNE_TABLE=os.devnull)
    cands = list(range(33))
    subprocess.run([sys.executable, "-c", _PACKED.format(root=root, ins=ins, attrs=json.dumps(attrs), out=out,
                                                          cands=cands)], env=env, check=True, timeout=120)
    r = np.load(out)
    for cand in cands:
        for what in ("single", "pair", "pair2") if group == 1 else ("single",):
            assert np.array_equal(r[f"{what}_{cand}_0"], r[f"{what}_{cand}_1"]), (what, cand)
    want = restate.conv(x, w, b, attrs["strides"], None, attrs["pads"], group, "NOTSET")
    compare(r["single_0_1"], np.where(want > 0, want, np.float32(0)).astype(F), what="packed FusedConv")
