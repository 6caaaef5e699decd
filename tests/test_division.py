"""The printed nests' division of an f32 value by a constant c (hipgen.cpp's
div_by_const, devfmt.hpp's pk_div_rc): the f64 product a * RN64(1/c)
rounded to f32 is the correctly rounded quotient.  Here numpy's float32
division (IEEE, correctly rounded) is the check, on sampled dividends of
every magnitude, the specials, and quotients that are exact midpoints of
the subnormal grid (where a wrong double rounding would show); the device's
own form is scanned over every f32 in tests/test_gpu_scalar.py."""
import numpy as np
import pytest

DIVISORS = [np.sqrt(2), np.sqrt(2 * np.pi), 3.0, 0.1, 6.0, 1.5, 7.0, 1234.5678, 1e-40, 3e30, -6.0, 11.3137085]


def via_rc(a, c):
    c32 = np.float32(c)
    rc = 1.0 / np.float64(c32)
    return (a.astype(np.float64) * rc).astype(np.float32)


@pytest.mark.parametrize("c", DIVISORS)
def test_sampled_dividends(c):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4028235e38, 1.1754944e-38], np.float32)
    a = np.concatenate([bits.view(np.float32), specials])
    with np.errstate(all="ignore"):
        want = a / np.float32(c)
        got = via_rc(a, c)
    same = (want.view(np.uint32) == got.view(np.uint32)) | (np.isnan(want) & np.isnan(got))
    assert same.all(), a[~same][:4]


@pytest.mark.parametrize("c", [6.0, 10.0, 12.0, 14.0, 18.0, 24.0])
def test_midpoint_quotients(c):
    """a = c * m for m an odd multiple of 2^-150 (a midpoint of the
    subnormal grid), wherever a is an f32 (c even times an odd part, so
    that a lies on the grid): the quotient must round to even exactly as
    the division does"""
    m = np.arange(1, 1 << 16, 2, dtype=np.float64) * 2.0 ** -150
    a64 = m * np.float64(np.float32(c))
    a = a64.astype(np.float32)
    a = a[a.astype(np.float64) == a64]
    assert a.size > 0
    with np.errstate(all="ignore"):
        want = a / np.float32(c)
    got = via_rc(a, c)
    assert (want.view(np.uint32) == got.view(np.uint32)).all()
