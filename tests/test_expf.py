"""The library's expf (mynah-slm_amd/csrc/mynah_expf.h), the exponential of
the decode step's softmax and SwiGLU sigmoid, against the C library's expf
(what the reference's f32 operators call, src/kernels.c:193-220).

On the CPU: the header compiled for the host (oracle/expf_pin.c), every
float in (-110, 90) — all finite inputs whose result is neither 0 nor
overflow — plus every 4096th bit pattern elsewhere (infinities, NaNs,
underflow and overflow ranges), bit for bit. On the GPU
(mynah_hip_expf_dev): every 61st float of the same range and the special
values, bit for bit against the C library.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PIN = C.CDLL(os.path.join(ROOT, "oracle", "libexpf_pin.so"))
PIN.orc_expf_sweep.restype = C.c_uint64
PIN.orc_expf_sweep.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_int,
                               C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)]
PIN.orc_mynah_expf.restype = C.c_float
PIN.orc_mynah_expf.argtypes = [C.c_float]
PIN.orc_libm_expf_array.restype = None
PIN.orc_libm_expf_array.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]


def bits(f: float) -> int:
    return struct.unpack("<I", struct.pack("<f", f))[0]


RANGES = [(0x00000000, bits(90.0) + 1), (0x80000000, bits(-110.0) + 1)]


def sweep(lo, hi, step):
    tested, first = C.c_uint64(0), C.c_uint32(0)
    bad = PIN.orc_expf_sweep(lo, hi, step, min(16, os.cpu_count() or 1), C.byref(tested),
                             C.byref(first))
    return int(bad), int(tested.value), int(first.value)


@pytest.mark.parametrize("lo,hi", RANGES, ids=["[0,90]", "[-110,0]"])
def test_every_float_of_the_softmax_range(lo, hi):
    bad, tested, first = sweep(lo, hi, 1)
    assert tested > 1_000_000_000
    assert bad == 0, f"{bad} of {tested} differ, first at 0x{first:08x}"


def test_the_rest_of_the_floats_sampled():
    bad, tested, first = sweep(bits(90.0), 0x100000000, 4096)
    assert bad == 0, f"first at 0x{first:08x}"
    bad, tested, first = sweep(bits(-110.0), 0x100000000, 4096)
    assert bad == 0, f"first at 0x{first:08x}"


def test_special_values():
    e = PIN.orc_mynah_expf
    assert e(float("-inf")) == 0.0 and e(float("inf")) == float("inf")
    assert np.isnan(e(float("nan")))
    assert e(0.0) == 1.0 and e(-0.0) == 1.0
    assert e(89.0) == float("inf") and e(-105.0) == 0.0
    assert 0.0 < e(-103.5) < 1e-44                    # a subnormal result


def host_expf(x: np.ndarray) -> np.ndarray:
    y = np.empty_like(x)
    PIN.orc_libm_expf_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


@pytest.mark.gpu
def test_device_expf_matches_the_c_library():
    import mynah_amd as M
    M.check(M.lib.mynah_hip_init(0), "init")
    u = np.concatenate([np.arange(lo, hi, 61, dtype=np.uint64) for lo, hi in RANGES])
    x = u.astype(np.uint32).view(np.float32)
    extra = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 88.5, 88.8, -103.5, -104.0, -1e-45,
                      1e-45, 3.4e38, -3.4e38], np.float32)
    x = np.concatenate([x, extra])
    print(f"[case] device expf over {x.size} floats", flush=True)
    xd = M.DeviceBuffer.from_array(x)
    yd = M.DeviceBuffer(x.nbytes)
    M.check(M.lib.mynah_hip_expf_dev(xd.ptr, yd.ptr, x.size, None), "expf_dev")
    M.sync()
    got = yd.download(np.float32, x.size)
    want = host_expf(x)
    same = got.view(np.uint32) == want.view(np.uint32)
    nan = np.isnan(got) & np.isnan(want)
    assert (same | nan).all(), f"{(~(same | nan)).sum()} differ, e.g. x={x[~(same | nan)][:4]}"
