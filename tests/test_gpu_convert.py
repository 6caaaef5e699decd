"""The device's edge conversion (presk_hip_convert) against the oracle's
restatement of the reference's Buf::of(to, b.to_f64()) (oracle/convert.c,
itself pinned to the reference's presk_convert): every pair of storage
types over every bf16, f16 and e8m15 code and the special and random f32 and
f64 values of tests/convert_cases.py -- bytes and guard identical, directly
and as a step of a recorded sequence replayed as a graph."""
import ctypes
import os

import numpy as np
import pytest

from presk_amd import hip
from tests.convert_cases import TYPES, WIDTH, source_bytes

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def oracle_convert(oracle_lib):
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "liboracle.so"))
    f = lib.po_convert
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    f.restype = ctypes.c_uint32
    return f


@pytest.mark.parametrize("frm", list(TYPES))
def test_device_edge_conversion(oracle_convert, frm):
    hip.init(0)
    src = source_bytes(frm)
    n = src.size // WIDTH[frm]
    d_src = hip.DeviceBuffer.of(src)
    for to in TYPES:
        want = np.zeros(n * WIDTH[to], np.uint8)
        wflag = oracle_convert(want.ctypes.data, TYPES[to], src.ctypes.data, TYPES[frm], n)
        out = hip.DeviceBuffer(want.size)
        flag = hip.DeviceBuffer(4)
        flag.zero()
        hip.check(hip.lib().presk_hip_convert(d_src.ptr, frm.encode(), out.ptr, to.encode(), n, flag.ptr, None))
        hip.sync()
        got = out.download(np.uint8, want.size)
        if got.tobytes() != want.tobytes():
            w = WIDTH[to]
            bad = np.nonzero((got.reshape(-1, w) != want.reshape(-1, w)).any(axis=1))[0]
            pytest.fail(f"{frm}->{to}: {bad.size} elements differ, first at {bad[:5]}")
        assert int(flag.download(np.uint32, 1)[0]) == wflag, (frm, to)


def test_conversion_in_a_graph(oracle_convert):
    """f32 -> bf16 -> f16 -> f32 as three steps of one recorded sequence,
    replayed three times as a graph"""
    hip.init(0)
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(100003) * 3000).astype(np.float32)
    want_b = np.zeros(x.size * 2, np.uint8)
    oracle_convert(want_b.ctypes.data, TYPES["bf16"], x.ctypes.data, TYPES["f32"], x.size)
    want_h = np.zeros(x.size * 2, np.uint8)
    oracle_convert(want_h.ctypes.data, TYPES["f16"], want_b.ctypes.data, TYPES["bf16"], x.size)
    want_f = np.zeros(x.size * 4, np.uint8)
    oracle_convert(want_f.ctypes.data, TYPES["f32"], want_h.ctypes.data, TYPES["f16"], x.size)
    a = hip.DeviceBuffer.of(x)
    b, h, f = hip.DeviceBuffer(x.size * 2), hip.DeviceBuffer(x.size * 2), hip.DeviceBuffer(x.size * 4)
    flag = hip.DeviceBuffer(4)
    flag.zero()
    L = hip.lib()
    bt = ctypes.c_void_p()
    hip.check(L.presk_hip_batch_create(ctypes.byref(bt)))
    hip.check(L.presk_hip_batch_add_convert(bt, a.ptr, b"f32", b.ptr, b"bf16", x.size, flag.ptr))
    hip.check(L.presk_hip_batch_add_convert(bt, b.ptr, b"bf16", h.ptr, b"f16", x.size, flag.ptr))
    hip.check(L.presk_hip_batch_add_convert(bt, h.ptr, b"f16", f.ptr, b"f32", x.size, flag.ptr))
    hip.check(L.presk_hip_batch_graph(bt))
    for _ in range(3):
        f.upload(np.full(x.size * 4, 0x5A, np.uint8))
        hip.sync()
        hip.check(L.presk_hip_batch_run(bt, None))
        hip.sync()
        assert b.download(np.uint8, x.size * 2).tobytes() == want_b.tobytes()
        assert h.download(np.uint8, x.size * 2).tobytes() == want_h.tobytes()
        assert f.download(np.uint8, x.size * 4).tobytes() == want_f.tobytes()
    L.presk_hip_batch_release(bt)
