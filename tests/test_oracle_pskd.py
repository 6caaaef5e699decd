"""The oracle's .psk.d leaf decode (oracle/convert.c: po_format_decode,
po_pskd_decode, po_pskd_idx) pinned by what fixes it independently of its
own formulas:

- binary16 described by its parameters against numpy's float16 on every code;
- the reference's own E4M3 codes of 480, -0.375, 2^-9 and -0
  (crates/presk-data/tests/data.rs:235-236: 0x7f, 0xac, 0x01, 0x80);
- E2M1's eight magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6 (crates/presk-format/
  src/lib.rs:141-143) and its largest finite number 6 (lib.rs:1638);
- the largest finite numbers and least positive numbers the reference's
  tests state (lib.rs:1629-1640): E4M3FN 448, E4M3 (saturating) 480 and
  2^-9, E5M2 57344; their NaN codes;
- bf16 and f32 as formats against their bit layouts (numpy), every bf16 code;
- encodings 0-2 are the edge conversion, which tests/test_oracle_convert.py
  pins against the reference's runtime;
- idx widening against numpy's little-endian integer views.
A dropped bias, a trailing-bit mask off by one or a sign left on a NaN
fails one of these."""
import ctypes
import math

import numpy as np
import pytest

from presk_amd import pskd


@pytest.fixture(scope="module")
def lib(oracle_lib):
    L = oracle_lib
    L.po_format_decode.restype = ctypes.c_double
    L.po_format_decode.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.po_pskd_decode.restype = ctypes.c_uint32
    L.po_pskd_decode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_size_t]
    L.po_pskd_idx.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    return L


def dec(lib, f: pskd.Format, code: int) -> float:
    return lib.po_format_decode(code, f.p, f.emin, f.emax, int(f.subnormals), pskd.SPECIALS.index(f.specials))


def decode_all(lib, f: pskd.Format, codes: np.ndarray, to: str = "f64") -> np.ndarray:
    """po_pskd_decode of the codes (as the file stores them) into `to`."""
    w = f.width
    src = np.zeros(codes.size * w, np.uint8)
    for b in range(w):
        src[b::w] = (codes >> np.uint64(8 * b)).astype(np.uint8)
    nb = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3}[to]
    dst = np.zeros(codes.size * nb, np.uint8)
    code = {"f64": 0, "f32": 1, "bf16": 2, "f16": 4, "e8m15": 5}[to]
    lib.po_pskd_decode(dst.ctypes.data, code, src.ctypes.data, 3, w, f.p, f.emin, f.emax, int(f.subnormals),
                       pskd.SPECIALS.index(f.specials), codes.size)
    return dst


def same(a: float, b: float) -> bool:
    return (math.isnan(a) and math.isnan(b)) or (a == b and math.copysign(1, a) == math.copysign(1, b))


def test_binary16_every_code(lib):
    codes = np.arange(1 << 16, dtype=np.uint64)
    got = decode_all(lib, pskd.F16, codes).view(np.float64)
    want = codes.astype(np.uint16).view(np.float16).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint64), want[~nan].view(np.uint64))
    # a NaN keeps its code's sign
    assert np.array_equal(np.signbit(got[nan]), codes[nan] >= 0x8000)


def test_e4m3_codes_of_the_reference(lib):
    f = pskd.E4M3_SATURATING
    for code, want in [(0x7F, 480.0), (0xAC, -0.375), (0x01, 2.0 ** -9), (0x80, -0.0)]:
        assert same(dec(lib, f, code), want), hex(code)
        assert f.encode(want) == code
    # every code finite, none NaN (specials none); 0xff is -480
    vals = [dec(lib, f, c) for c in range(256)]
    assert all(math.isfinite(v) for v in vals) and max(vals) == 480.0 and min(vals) == -480.0


def test_e2m1_magnitudes(lib):
    f = pskd.E2M1
    assert f.bits == 4
    got = sorted({abs(dec(lib, f, c)) for c in range(16)})
    assert got == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    assert [dec(lib, f, c) for c in (0b0111, 0b1111)] == [6.0, -6.0]


@pytest.mark.parametrize("f,maxf,minp", [(pskd.E4M3FN, 448.0, 2.0 ** -9), (pskd.E4M3_SATURATING, 480.0, 2.0 ** -9),
                                         (pskd.E5M2, 57344.0, 2.0 ** -16), (pskd.F16, 65504.0, 2.0 ** -24)])
def test_extremes_the_reference_states(lib, f, maxf, minp):
    vals = [dec(lib, f, c) for c in range(1 << f.bits)]
    fin = [v for v in vals if math.isfinite(v)]
    assert max(fin) == maxf and min(v for v in fin if v > 0) == minp
    if f.specials == "nan":
        assert math.isnan(dec(lib, f, 0x7F)) and math.isnan(dec(lib, f, 0xFF)) and dec(lib, f, 0x7E) == 448.0
    if f.specials == "ieee":
        top = ((1 << f.ebits) - 1) << (f.p - 1)
        assert dec(lib, f, top) == math.inf and math.isnan(dec(lib, f, top | 1))


def test_bf16_and_f32_as_formats(lib):
    codes = np.arange(1 << 16, dtype=np.uint64)
    got = decode_all(lib, pskd.Format(8, -126, 127), codes).view(np.float64)
    with np.errstate(invalid="ignore"):
        want = (codes.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], want[~nan])
    rng = np.random.default_rng(5)
    c32 = np.concatenate([rng.integers(0, 2 ** 32, 20000, dtype=np.uint64),
                          np.array([0, 1, 0x807FFFFF, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x00800000], np.uint64)])
    got = decode_all(lib, pskd.Format(24, -126, 127), c32).view(np.float64)
    with np.errstate(invalid="ignore"):
        want = c32.astype(np.uint32).view(np.float32).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], want[~nan])


def test_host_format_codec_agrees_with_the_oracle(lib):
    """The writer's Format.encode/decode (presk_amd/pskd.py) against the
    oracle's decode: every code of each 8- and 16-bit format decodes alike,
    and every finite value encodes back to its code (the canonical one)."""
    for f in (pskd.E4M3FN, pskd.E4M3_SATURATING, pskd.E5M2, pskd.E2M1, pskd.F16):
        for c in range(1 << f.bits):
            o = dec(lib, f, c)
            assert same(o, f.decode(c)), (f, c)
            if math.isfinite(o):
                c2 = f.encode(o)
                assert c2 is not None and same(f.decode(c2), o)


def test_into_storage_types_rounds_as_the_conversion(lib):
    """A described format's decode into a storage type equals decoding to
    f64 and converting (po_convert, pinned against the reference runtime)."""
    conv = lib.po_convert
    conv.restype = ctypes.c_uint32
    conv.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    f = pskd.Format(20, -254, 255).check()    # wider than f32's range: rounding and overflow both happen
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 1 << f.bits, 50000, dtype=np.uint64)
    f64 = decode_all(lib, f, codes, "f64")
    for to, tc, nb in [("f32", 1, 4), ("bf16", 2, 2), ("f16", 4, 2), ("e8m15", 5, 3)]:
        got = decode_all(lib, f, codes, to)
        want = np.zeros(codes.size * nb, np.uint8)
        conv(want.ctypes.data, tc, f64.ctypes.data, 0, codes.size)
        assert got.tobytes() == want.tobytes(), to


@pytest.mark.parametrize("width,dt", [(1, np.uint8), (2, np.uint16), (4, np.uint32), (8, np.uint64)])
def test_idx_widening(lib, width, dt):
    rng = np.random.default_rng(width)
    v = rng.integers(0, np.iinfo(dt).max, 1000, dtype=dt, endpoint=True)
    out = np.zeros(v.size, np.int64)
    src = np.ascontiguousarray(v.astype("<" + np.dtype(dt).str[1:]))   # held: the call reads it
    lib.po_pskd_idx(out.ctypes.data, src.ctypes.data, width, v.size)
    assert np.array_equal(out.view(np.uint64), v.astype(np.uint64))
