"""CPU: pin the oracle before trusting it.

Checks (no GPU):
  * the reference library (oracle/_ref) reproduces the reference's own
    known-answer values (tests/golden/known_answers.json, transcribed from
    test/kernels_test.cpp and test/hip_kernels_test.cpp);
  * the numpy restatement (oracle/restate.py) agrees with the reference rows on
    seeded random cases and on the same known answers;
  * properties the mathematics fixes (transpose identities, linearity,
    brute-force loops on tiny inputs), chosen so that a dropped bias, a swapped
    transpose or an off-by-one pad fails.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import ref, restate
from rowcheck import compare, randn, run_ref, uniform

F, I = np.float32, np.int64
GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"


def _load_golden():
    return json.loads(GOLDEN.read_text())["cases"]


def _arr(spec):
    return np.array(spec["data"], dtype={"f32": F, "i64": I, "bool": np.bool_}[spec["dtype"]]).reshape(spec["shape"])


@pytest.mark.parametrize("case", _load_golden(), ids=lambda c: c["id"])
def test_reference_reproduces_known_answers(case):
    inputs = [None if s is None else _arr(s) for s in case["inputs"]]
    specs = [(tuple(o["shape"]), {"f32": F, "i64": I, "bool": np.bool_}[o["dtype"]]) for o in case["outputs"]]
    outs, err = run_ref(case["op"], inputs, specs, case.get("attrs"), schema_version=case.get("schema_version", 0))
    assert err is None, err
    for got, want in zip(outs, case["outputs"]):
        compare(got, _arr(want), rtol=case.get("rtol", 0.0), atol=case.get("atol", 0.0), what=case["id"])


def _golden(op):
    return [c for c in _load_golden() if c["op"] == op]


@pytest.mark.parametrize("case", _golden("Gemm"), ids=lambda c: c["id"])
def test_restate_gemm_known_answers(case):
    ins = [_arr(s) for s in case["inputs"]]
    a = case.get("attrs", {})
    got = restate.gemm(ins[0], ins[1], ins[2] if len(ins) > 2 else None, a.get("transA", 0), a.get("transB", 0),
                       a.get("alpha", 1.0), a.get("beta", 1.0))
    compare(got, _arr(case["outputs"][0]), rtol=0, atol=0, what=case["id"])


@pytest.mark.parametrize("case", _golden("Conv"), ids=lambda c: c["id"])
def test_restate_conv_known_answers(case):
    ins = [_arr(s) for s in case["inputs"]]
    a = case.get("attrs", {})
    got = restate.conv(ins[0], ins[1], ins[2] if len(ins) > 2 else None, a.get("strides"), a.get("dilations"),
                       a.get("pads"), a.get("group", 1), a.get("auto_pad", "NOTSET"))
    compare(got, _arr(case["outputs"][0]), rtol=0, atol=0, what=case["id"])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_restate_gemm_matches_reference(ta, tb):
    m, n, k = 13, 11, 29
    a = uniform((k, m) if ta else (m, k), seed=1)
    b = uniform((n, k) if tb else (k, n), seed=2)
    c = uniform((m, n), seed=3)
    attrs = {"transA": ta, "transB": tb, "alpha": 0.5, "beta": 2.0}
    outs, err = run_ref("Gemm", [a, b, c], [((m, n), F)], attrs)
    assert err is None
    compare(restate.gemm(a, b, c, ta, tb, 0.5, 2.0), outs[0], rtol=1e-6, atol=1e-6, what="gemm")
    # A plausible mistake -- ignoring transB -- must fail this comparison.
    if tb and n == k:
        assert not np.allclose(restate.gemm(a, b.T.copy(), c, ta, 0, 0.5, 2.0), outs[0])


@pytest.mark.parametrize("sa,sb", [((3, 4, 5), (5, 2)), ((2, 1, 3, 4), (5, 4, 6)), ((4,), (4, 3)), ((2, 4), (4,))])
def test_restate_matmul_matches_reference(sa, sb):
    a, b = uniform(sa, seed=4), uniform(sb, seed=5)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    outs, err = run_ref("MatMul", [a, b], [(want.shape, F)])
    assert err is None
    compare(restate.matmul(a, b), outs[0], rtol=1e-6, atol=1e-6, what="matmul")


CONV = [
    ((1, 3, 8, 9), (4, 3, 3, 3), dict(pads=[1, 1, 1, 1])),
    ((2, 4, 9, 9), (6, 2, 3, 2), dict(group=2, strides=[2, 1], dilations=[1, 2], pads=[1, 0, 2, 1])),
    ((1, 2, 7), (3, 2, 3), dict(auto_pad="SAME_UPPER", strides=[2])),
    ((1, 2, 4, 5, 5), (2, 2, 2, 3, 3), dict(pads=[0, 1, 1, 1, 0, 1])),
    ((1, 2, 6, 6), (2, 2, 3, 3), dict(auto_pad="SAME_LOWER", strides=[2, 2])),
]


@pytest.mark.parametrize("xs,ws,a", CONV)
def test_restate_conv_matches_reference(xs, ws, a):
    x, w, b = randn(xs, seed=6), randn(ws, seed=7), randn((ws[0],), seed=8)
    want = restate.conv(x, w, b, a.get("strides"), a.get("dilations"), a.get("pads"), a.get("group", 1),
                        a.get("auto_pad", "NOTSET"))
    outs, err = run_ref("Conv", [x, w, b], [(want.shape, F)], a)
    assert err is None, err
    compare(want, outs[0], rtol=1e-6, atol=1e-6, what="conv")


def test_restate_conv_brute_force_tiny():
    """Direct 7-loop evaluation of the ONNX definition on a tiny case."""
    x, w, b = randn((1, 2, 5, 4), seed=9), randn((3, 2, 2, 3), seed=10), randn((3,), seed=11)
    s, d, p = [2, 1], [1, 2], [1, 2, 0, 1]
    got = restate.conv(x, w, b, s, d, p)
    oh = (5 + 1 + 0 - 2) // 2 + 1
    ow = (4 + 2 + 1 - 5) // 1 + 1
    want = np.zeros((1, 3, oh, ow))
    for m in range(3):
        for i in range(oh):
            for j in range(ow):
                acc = float(b[m])
                for c in range(2):
                    for kh in range(2):
                        for kw in range(3):
                            ih, iw = i * 2 - 1 + kh, j - 2 + kw * 2
                            if 0 <= ih < 5 and 0 <= iw < 4:
                                acc += float(x[0, c, ih, iw]) * float(w[m, c, kh, kw])
                want[0, m, i, j] = acc
    compare(got, want.astype(F), rtol=1e-6, atol=1e-6, what="brute force")


def test_reference_rows_present():
    for op in ["Gemm", "MatMul", "Conv", "Relu", "Add", "MaxPool", "GlobalAveragePool", "Softmax", "TopK"]:
        assert ref.has_row(op)
