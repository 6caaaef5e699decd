"""Device dropout masks (presk_hip_dropout_mask) against the oracle's
restatement of the host's (oracle/rng.c, itself pinned to the reference's
runtime and golden draws): every byte, for every storage type, ragged and
large sizes, several rates; the refusal of a rate outside [0, 1); and a
recorded sequence whose graph, replayed after the host writes a new key to
the device, draws the new key's mask."""
import ctypes

import numpy as np
import pytest

from presk_amd import hip, keys
from tests.test_oracle_rng import lib

pytestmark = pytest.mark.gpu

CODES = {"f64": 0, "f32": 1, "bf16": 2, "f16": 4, "e8m15": 5}


def oracle_mask(key: bytes, rate, ty, n):
    out = np.zeros(max(n, 1) * hip.STORAGE_BYTES[ty], np.uint8)
    lib().po_dropout_mask((ctypes.c_uint8 * 32)(*key), rate, CODES[ty], n, out.ctypes.data)
    return out[: n * hip.STORAGE_BYTES[ty]]


def device_key(key: bytes):
    b = hip.DeviceBuffer(32)
    b.upload(np.frombuffer(key, np.uint8))
    return b


@pytest.mark.parametrize("ty", list(CODES))
def test_mask_bits(ty):
    hip.init(0)
    k = keys.child(keys.from_seed(11), 4)
    kb = device_key(k)
    for n in (1, 7, 8, 9, 65_537, 3_000_001):
        for rate in (0.0, 0.2, 0.5, 0.9):
            print(f"[dropout] {ty} n={n} rate={rate}", flush=True)
            nb = n * hip.STORAGE_BYTES[ty]
            out = hip.DeviceBuffer(nb)
            out.upload(np.full(nb, 0xAB, np.uint8))
            hip.check(hip.lib().presk_hip_dropout_mask(kb.ptr, rate, ty.encode(), n, out.ptr, None))
            hip.sync()
            got = out.download(np.uint8, nb)
            assert got.tobytes() == oracle_mask(k, rate, ty, n).tobytes(), (ty, n, rate)


def test_rate_outside_range_is_refused():
    hip.init(0)
    kb = device_key(keys.from_seed(1))
    out = hip.DeviceBuffer(64)
    for rate in (1.0, -0.1, float("nan")):
        rc = hip.lib().presk_hip_dropout_mask(kb.ptr, rate, b"f32", 16, out.ptr, None)
        assert rc != 0
        assert hip.lib().presk_hip_last_error().decode().startswith(("E7001", "E10001"))


def test_graph_replay_draws_the_current_key():
    hip.init(0)
    L = hip.lib()
    k1, k2 = keys.from_seed(21), keys.from_seed(22)
    kb = device_key(k1)
    n = 100_003
    out = hip.DeviceBuffer(n * 2)
    b = ctypes.c_void_p()
    hip.check(L.presk_hip_batch_create(ctypes.byref(b)))
    try:
        hip.check(L.presk_hip_batch_add_dropout(b, kb.ptr, 0.2, b"bf16", n, out.ptr))
        hip.check(L.presk_hip_batch_graph(b))
        hip.check(L.presk_hip_batch_run(b, None))
        hip.sync()
        assert out.download(np.uint8, 2 * n).tobytes() == oracle_mask(k1, 0.2, "bf16", n).tobytes()
        kb.upload(np.frombuffer(k2, np.uint8))
        hip.check(L.presk_hip_batch_run(b, None))
        hip.sync()
        assert out.download(np.uint8, 2 * n).tobytes() == oracle_mask(k2, 0.2, "bf16", n).tobytes()
    finally:
        L.presk_hip_batch_release(b)
