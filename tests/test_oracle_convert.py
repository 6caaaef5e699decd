"""The oracle's edge conversion (oracle/convert.c) against the reference's
own runtime, presk_convert (crates/presk-export-c/c/presk_rt.c, built into
oracle/_ref): every pair of storage types, every bf16, f16 and e8m15 code,
and the special and random f32 and f64 values of tests/convert_cases.py --
bytes and the overflow guard identical."""
import ctypes
import os

import numpy as np
import pytest

from tests.convert_cases import TYPES, WIDTH, source_bytes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "libpresk_rt.so")


def _lib(path, fn):
    lib = ctypes.CDLL(path)
    f = getattr(lib, fn)
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    f.restype = ctypes.c_uint32
    return f


def run(f, src, frm, to):
    n = src.size // WIDTH[frm]
    dst = np.zeros(n * WIDTH[to], np.uint8)
    flag = f(dst.ctypes.data, TYPES[to], src.ctypes.data, TYPES[frm], n)
    return dst, flag


@pytest.fixture(scope="module")
def fns(oracle_lib):
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libpresk_rt.so is built only where the reference sources are")
    mine = _lib(os.path.join(ROOT, "oracle", "liboracle.so"), "po_convert")
    return mine, _lib(REF, "presk_convert")


@pytest.mark.parametrize("frm", list(TYPES))
@pytest.mark.parametrize("to", list(TYPES))
def test_edge_conversion_matches_reference(fns, frm, to):
    mine, ref = fns
    src = source_bytes(frm)
    got, gf = run(mine, src, frm, to)
    want, wf = run(ref, src, frm, to)
    assert gf == wf
    if got.tobytes() != want.tobytes():
        w = WIDTH[to]
        bad = np.nonzero((got.reshape(-1, w) != want.reshape(-1, w)).any(axis=1))[0]
        pytest.fail(f"{frm}->{to}: {bad.size} elements differ, first at {bad[:5]}")
