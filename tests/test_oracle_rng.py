"""The oracle's restatement of Presk's keys and draws (oracle/rng.c) pinned:
against the reference's own golden numbers -- the first four normals of
Key::from_seed(0) and an FNV-1a fold of the next 100 000
(crates/presk-interp/src/key.rs:85-93, drawn by rand_chacha 0.9 and the
`libm` crate's log and cos; here the stream is the oracle's and log/cos the
reference's own C, oracle/_ref) -- and against the reference's C runtime
(crates/presk-export-c/c/presk_rt.c, built into oracle/_ref): key splits,
children and seeds, and the uniform draws of random keys word for word."""
import ctypes
import math
import os

import numpy as np
import pytest

from oracle import cexec

HERE = os.path.join(os.path.dirname(cexec.__file__))
REF = os.path.join(HERE, "_ref", "libpresk_rt.so")
u8x32 = ctypes.c_uint8 * 32


def lib():
    L = ctypes.CDLL(os.path.join(HERE, "liboracle.so"))
    L.po_uniform01_at.restype = ctypes.c_double
    L.po_uniform01_at.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    L.po_key_split.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    L.po_key_child.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    L.po_key_from_seed.argtypes = [ctypes.c_uint64, ctypes.c_void_p]
    L.po_dropout_mask.argtypes = [ctypes.c_void_p, ctypes.c_double, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p]
    return L


def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref is built only where the reference's sources are")
    R = ctypes.CDLL(REF)
    R.presk_log.restype = R.presk_cos.restype = ctypes.c_double
    R.presk_log.argtypes = R.presk_cos.argtypes = [ctypes.c_double]
    R.presk_uniform01.restype = ctypes.c_double
    R.presk_key_from_seed.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    R.presk_key_split.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    R.presk_key_child.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    return R


def key_from_seed(L, s):
    k = u8x32()
    L.po_key_from_seed(s, k)
    return k


def test_golden_normals_of_key_seed_zero():
    """key.rs:85-93: the normals Key::from_seed(0) draws, Box-Muller in f64
    over uniform01 (a zero u1 redrawn), with the reference's log and cos"""
    L, R = lib(), ref()
    k = key_from_seed(L, 0)
    e = 0

    def uni():
        nonlocal e
        u = L.po_uniform01_at(k, e)
        e += 1
        return u

    def normal():
        u1 = uni()
        while u1 <= 0.0:
            u1 = uni()
        u2 = uni()
        return math.sqrt(-2.0 * R.presk_log(u1)) * R.presk_cos(2.0 * math.pi * u2)

    bits = lambda x: int(np.float64(x).view(np.uint64))
    first = [bits(normal()) for _ in range(4)]
    assert first == [0x3feac568a525e1d1, 0xbfc884e0b5405abc, 0xbff1feb45f60e89a, 0x3fee552e3fbd0476]
    h = 0xcbf29ce484222325
    for _ in range(100_000):
        h = ((h ^ bits(normal())) * 0x00000100000001b3) & 0xFFFFFFFFFFFFFFFF
    assert h == 0xf10af503abdab221


def test_keys_and_draws_are_the_reference_runtimes():
    L, R = lib(), ref()
    rng = np.random.default_rng(0)
    for seed in [0, 1, 42, 0xdeadbeef, 2**64 - 1]:
        a, b = key_from_seed(L, seed), u8x32()
        R.presk_key_from_seed(b, seed)
        assert bytes(a) == bytes(b), seed
    # the reference's generator state (presk_rng: 8 key words, a counter, 64
    # result words, an index) as opaque storage
    state = (ctypes.c_uint8 * 512)()
    for _ in range(6):
        k = u8x32(*rng.integers(0, 256, 32).tolist())
        for l in (0, 1, 2, 7):
            a, b = u8x32(), u8x32()
            L.po_key_split(k, l, a)
            R.presk_key_split(k, l, b)
            assert bytes(a) == bytes(b)
        for t in (0, 1, 5, 2**40 + 3):
            a, b = u8x32(), u8x32()
            L.po_key_child(k, t, a)
            R.presk_key_child(k, t, b)
            assert bytes(a) == bytes(b)
        R.presk_rng_from_seed(state, k)
        for e in range(3000):
            assert L.po_uniform01_at(k, e) == R.presk_uniform01(state), e


@pytest.mark.parametrize("code,ty", [(1, np.float32), (2, np.uint16), (4, np.uint16)])
def test_dropout_mask_is_kept_draws_scaled(code, ty):
    """element e is 1/(1-p) where draw e < 1-p, 0 elsewhere, rounded once"""
    L = lib()
    k = key_from_seed(L, 7)
    n, p = 10_001, 0.2
    out = np.zeros(n, ty)
    L.po_dropout_mask(k, p, code, n, out.ctypes.data)
    u = np.array([L.po_uniform01_at(k, e) for e in range(n)])
    want = np.where(u < 1 - p, 1 / (1 - p), 0.0)
    if code == 1:
        assert np.array_equal(out, want.astype(np.float32))
    else:
        from tests import fmt
        assert np.array_equal(out, fmt.encode(want.astype(np.float32), "bf16" if code == 2 else "f16"))
    assert abs(np.mean(u < 1 - p) - 0.8) < 0.02


def test_host_keys_are_the_oracles():
    """presk_amd/keys.py (the product's host-side derivation) against the
    oracle's restatement"""
    from presk_amd import keys
    L = lib()
    for seed in [0, 3, 2**63 + 5]:
        k = keys.from_seed(seed)
        assert k == bytes(key_from_seed(L, seed))
        kb = u8x32(*k)
        for l, part in enumerate(keys.split(k, 3)):
            o = u8x32()
            L.po_key_split(kb, l, o)
            assert part == bytes(o)
        for t in (0, 9, 2**33):
            o = u8x32()
            L.po_key_child(kb, t, o)
            assert keys.child(k, t) == bytes(o)
