"""GPU: nert_hip_topk_f32_noalloc, the allocation-free TopK entry point,
through the C-ABI against nert_hip_topk_f32 on the same inputs (bit-exact
values and indices), two calls in a row with the second one smaller, plus
the small-row path and a request beyond the fixed scratch (rejected, nothing
launched)."""

import ctypes as C

import numpy as np
import pytest

from nert_amd import device
from nert_amd.device import DeviceArray

pytestmark = pytest.mark.gpu


def _bind():
    L = device.lib()
    for name in ("nert_hip_topk_f32", "nert_hip_topk_f32_noalloc"):
        getattr(L, name).argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                     C.c_void_p]
    return L


def _topk(entry, x: np.ndarray, k: int):
    outer, dim = x.shape
    dx = DeviceArray.from_host(x)
    vals = DeviceArray((outer, k), np.float32)
    idx = DeviceArray((outer, k), np.int64)
    rc = getattr(_bind(), entry)(dx.ptr, vals.ptr, idx.ptr, outer, dim, 1, k, None)
    if rc != 0:
        return None, None, device.last_error()
    device.synchronize()
    return vals.to_host(), idx.to_host(), None


def _scores(rows, dim, seed):
    rng = np.random.default_rng(seed)
    x = rng.random((rows, dim), dtype=np.float32)
    x[:, ::7] = np.float32(0.5)  # heavy ties: the lower index must win
    return x


@pytest.mark.parametrize("rows,dim,k", [(8, 672000, 300), (3, 100000, 37)])
def test_noalloc_topk_matches_topk_twice(gpu, rows, dim, k):
    """The detector's [8, 672000] K=300, then a smaller call on the same
    scratch: both bit-identical to the allocating entry point."""
    for r, d, kk, seed in ((rows, dim, k, 1), (max(1, rows // 2), dim // 3, max(1, k // 3), 2)):
        x = _scores(r, d, seed)
        want_v, want_i, err = _topk("nert_hip_topk_f32", x, kk)
        assert err is None, err
        got_v, got_i, err = _topk("nert_hip_topk_f32_noalloc", x, kk)
        assert err is None, err
        assert np.array_equal(got_v, want_v) and np.array_equal(got_i, want_i), (r, d, kk)


def test_noalloc_topk_small_rows(gpu):
    x = _scores(64, 3000, 3)
    want_v, want_i, _ = _topk("nert_hip_topk_f32", x, 50)
    got_v, got_i, err = _topk("nert_hip_topk_f32_noalloc", x, 50)
    assert err is None and np.array_equal(got_v, want_v) and np.array_equal(got_i, want_i)


def test_noalloc_topk_rejects_oversized_request(gpu):
    # 4096 rows of 8192 with k = 2048: 4096 * (16 * 2048 + 3072) bytes > 4 MiB.
    x = np.zeros((4096, 8192), np.float32)
    _, _, err = _topk("nert_hip_topk_f32_noalloc", x, 2048)
    assert err is not None and "scratch" in err
    # The allocating entry point still serves it.
    v, i, err = _topk("nert_hip_topk_f32", x[:2], 2048)
    assert err is None and np.array_equal(i[0], np.arange(2048))
