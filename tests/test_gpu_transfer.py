"""GPU: host<->device transfers through the C-ABI (nert_hip_memcpy_h2d/d2h,
the HipDevice Transfer of src/hip_device.cpp:70-89).

Pageable copies of 1 MiB or more go through pinned bounce buffers in pieces
of 1, 2, then 4 MiB dealt to 2 host threads; the sizes below cover the
unstaged path, a single piece, both lanes, ragged tails, and more pieces than
the lanes' slots (so every slot is reused). Each staged direction is checked against the
unstaged path of the other (NERT_HIP_STAGING=0), with odd byte offsets on
both the host and the device side. Bit-exact: these are byte copies."""

import os

import numpy as np
import pytest

from nert_amd import abi, device
from nert_amd.device import DeviceArray, PinnedArray, check, lib

pytestmark = pytest.mark.gpu
NERT_UN_NEG = 10  # enum nert_unary_op in include/nert_hip.h

MIB = 1 << 20
SIZES = [1, 4096, MIB - 1, MIB, 4 * MIB, 5 * MIB + 3, 16 * MIB, 41 * MIB + 12]


def _h2d(dst_ptr, host, staged):
    os.environ["NERT_HIP_STAGING"] = "1" if staged else "0"
    try:
        check(lib().nert_hip_memcpy_h2d(dst_ptr, host.ctypes.data, host.nbytes), "h2d")
    finally:
        os.environ.pop("NERT_HIP_STAGING", None)


def _d2h(host, src_ptr, staged):
    os.environ["NERT_HIP_STAGING"] = "1" if staged else "0"
    try:
        check(lib().nert_hip_memcpy_d2h(host.ctypes.data, src_ptr, host.nbytes), "d2h")
    finally:
        os.environ.pop("NERT_HIP_STAGING", None)


@pytest.mark.parametrize("nbytes", SIZES)
@pytest.mark.parametrize("staged_h2d,staged_d2h", [(True, False), (False, True), (True, True)])
def test_transfer_round_trip(gpu, nbytes, staged_h2d, staged_d2h):
    rng = np.random.default_rng(nbytes)
    buf = DeviceArray((nbytes + 8,), np.uint8)
    try:
        src_store = rng.integers(0, 256, nbytes + 3, dtype=np.uint8)
        src = src_store[3:]  # host source not 16-byte aligned
        dst_ptr = buf.ptr + 5  # device destination not aligned either
        _h2d(dst_ptr, src, staged_h2d)
        out_store = np.full(nbytes + 7, 0xA5, np.uint8)
        out = out_store[7:]
        _d2h(out, dst_ptr, staged_d2h)
        assert np.array_equal(out, src)
        assert np.all(out_store[:7] == 0xA5)
    finally:
        buf.close()


def test_transfer_pinned_host_goes_direct(gpu):
    """A pinned host buffer (nert_hip_host_alloc) takes the direct DMA path
    and round-trips the same bytes."""
    n = 9 * MIB + 1
    pinned = PinnedArray((n,), np.uint8)
    host = pinned.array
    host[:] = np.random.default_rng(7).integers(0, 256, n, dtype=np.uint8)
    buf = DeviceArray((n,), np.uint8)
    try:
        _h2d(buf.ptr, host, True)
        back = np.empty(n, np.uint8)
        _d2h(back, buf.ptr, False)
        assert np.array_equal(back, host)
        host[:] = 0
        _d2h(host, buf.ptr, True)
        assert np.array_equal(back, host)
    finally:
        buf.close()
        pinned.close()


def test_transfer_follows_queued_kernels(gpu):
    """A staged D2H copy waits for work already queued on the layer stream;
    a staged H2D copy lands before later launches read it."""
    x = np.random.default_rng(3).standard_normal(3 * MIB).astype(np.float32)  # 12 MiB
    a = DeviceArray.from_host(x)
    y = DeviceArray(x.shape, np.float32)
    try:
        check(lib().nert_hip_unary(NERT_UN_NEG, abi.F32, a.ptr, y.ptr, x.size, 0.0, 0.0, None), "neg")
        got = np.empty_like(x)
        _d2h(got, y.ptr, True)
        assert np.array_equal(got, -x)
        x2 = x * 2
        _h2d(a.ptr, x2, True)
        check(lib().nert_hip_unary(NERT_UN_NEG, abi.F32, a.ptr, y.ptr, x.size, 0.0, 0.0, None), "neg")
        _d2h(got, y.ptr, True)
        assert np.array_equal(got, -x2)
    finally:
        a.close()
        y.close()
    device.synchronize()
