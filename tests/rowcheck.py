"""Row parity harness: run one node on the reference CpuDevice (oracle/_ref)
and on the gfx950 HipDevice, then compare.

Mirrors the reference's own HIP parity tests (test/hip_kernels_test.cpp:35-40
compare HIP against CpuDevice), with a stricter bar: integer, bool and index
outputs must be bit-identical; float32 outputs must satisfy
|hip - ref| <= atol + rtol * |ref| with rtol = atol = 1e-4 unless a test says
otherwise (NaN must match NaN). When the reference row throws, the HIP row
must throw the same InferenceException message.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np

from nert_amd import abi
from nert_amd.device import DeviceArray, NertError, run_node
from oracle import ref

RTOL = 1e-4
ATOL = 1e-4


def run_ref(op: str, inputs: Sequence[np.ndarray | None], out_specs: Sequence[tuple[Sequence[int], Any]],
            attrs: dict[str, Any] | None = None, name: str = "n", schema_version: int = 0):
    outs = [np.zeros(shape, dtype) for shape, dtype in out_specs]
    inputs = [None if x is None else np.asarray(x, order="C") for x in inputs]
    try:
        ref.run_node(op, inputs, outs, attrs, name, schema_version)
    except ref.RefError as e:
        return None, e
    return outs, None


def run_hip(op: str, inputs: Sequence[np.ndarray | None], out_specs: Sequence[tuple[Sequence[int], Any]],
            attrs: dict[str, Any] | None = None, name: str = "n", schema_version: int = 0):
    dev_in = [None if x is None else DeviceArray.from_host(np.asarray(x, order="C")) for x in inputs]
    dev_out = [DeviceArray.from_host(np.zeros(shape, dtype)) for shape, dtype in out_specs]
    try:
        run_node(op, dev_in, dev_out, attrs, name, schema_version)
    except NertError as e:
        return None, e
    return [d.to_host() for d in dev_out], None


def compare(hip: np.ndarray, want: np.ndarray, rtol: float = RTOL, atol: float = ATOL, what: str = "") -> None:
    assert hip.shape == want.shape, f"{what}: shape {hip.shape} != {want.shape}"
    assert hip.dtype == want.dtype, f"{what}: dtype {hip.dtype} != {want.dtype}"
    if want.dtype == np.float32:
        h = hip.astype(np.float64)
        r = want.astype(np.float64)
        nan_h, nan_r = np.isnan(h), np.isnan(r)
        assert np.array_equal(nan_h, nan_r), f"{what}: NaN positions differ"
        finite = ~nan_r
        inf_r = np.isinf(r) & finite
        assert np.array_equal(h[inf_r], r[inf_r]), f"{what}: infinities differ"
        ok = finite & ~inf_r
        diff = np.abs(h[ok] - r[ok])
        bound = atol + rtol * np.abs(r[ok])
        if diff.size:
            worst = int(np.argmax(diff - bound))
            assert np.all(diff <= bound), (
                f"{what}: {int(np.sum(diff > bound))} of {diff.size} elements outside "
                f"atol {atol} + rtol {rtol}; worst |d|={diff[worst]:.3e} at ref={r[ok][worst]:.6g}")
    else:
        if not np.array_equal(hip, want):
            bad = np.argwhere(hip != want)
            raise AssertionError(f"{what}: {len(bad)} elements differ (not bit-exact); first at {bad[0].tolist()}: "
                                 f"hip={hip[tuple(bad[0])]} ref={want[tuple(bad[0])]}")


def assert_parity(op: str, inputs: Sequence[np.ndarray | None], out_specs: Sequence[tuple[Sequence[int], Any]],
                  attrs: dict[str, Any] | None = None, name: str = "n", schema_version: int = 0,
                  rtol: float = RTOL, atol: float = ATOL, compare_outputs: Sequence[int] | None = None):
    """Runs the node on both devices and asserts parity; returns the HIP outputs.

    The case must be one the reference accepts (a rejected node would make
    the comparison vacuous); rejections are checked with assert_same_error."""
    want, ref_err = run_ref(op, inputs, out_specs, attrs, name, schema_version)
    assert ref_err is None, f"{op}: the reference rejects this case: {ref_err}"
    got, hip_err = run_hip(op, inputs, out_specs, attrs, name, schema_version)
    assert hip_err is None, f"{op}: HIP threw but the reference did not: {hip_err}"
    idx = range(len(out_specs)) if compare_outputs is None else compare_outputs
    for i in idx:
        compare(got[i], want[i], rtol, atol, what=f"{op} output {i}")
    return got


def assert_same_error(op: str, inputs, out_specs, attrs=None, name: str = "bad_node", schema_version: int = 0) -> str:
    """Both devices must reject the node with the same message naming node and op."""
    _, ref_err = run_ref(op, inputs, out_specs, attrs, name, schema_version)
    _, hip_err = run_hip(op, inputs, out_specs, attrs, name, schema_version)
    assert ref_err is not None, f"{op}: reference accepted the node"
    assert hip_err is not None, f"{op}: HIP accepted the node the reference rejects ({ref_err})"
    assert ref_err.status == abi.INFERENCE_ERROR and hip_err.status == abi.INFERENCE_ERROR, (ref_err, hip_err)
    assert hip_err.message == ref_err.message, f"{op}:\n hip: {hip_err}\n ref: {ref_err}"
    assert name in hip_err.message and op in hip_err.message
    return hip_err.message


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def randn(shape, seed=0, scale=1.0) -> np.ndarray:
    return np.asarray(rng(seed).standard_normal(shape) * scale, dtype=np.float32)


def uniform(shape, lo=-1.0, hi=1.0, seed=0) -> np.ndarray:
    return np.asarray(rng(seed).uniform(lo, hi, shape), dtype=np.float32)
