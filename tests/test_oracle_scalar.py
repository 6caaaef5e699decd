"""The oracle's conversions and libm against the reference's own C runtime.

tests/golden/digests.json holds, per function, the digest of every block of
its domain computed from crates/presk-export-c/c/presk_rt.h and presk_libm.c
(tests/golden/make_golden.py).  Every block of the oracle's restatement must
give the same digest: every f32 input for expf/logf/tanhf/erff and the
narrowings, every code for the widenings; the f64 functions over a sample
of 2^24 arguments and at their special arguments.  Independent checks beside
the reference's: numpy's IEEE binary16 rounding, closed forms, and the f64
functions within an ulp or two of numpy's (another libm) away from their
branch points.
"""
import ctypes

import numpy as np
import pytest

from tests.golden import spec


@pytest.mark.parametrize("name", list(spec.FUNCTIONS))
def test_oracle_matches_reference_everywhere(name, oracle_lib, golden):
    g = golden["functions"][name]
    fid, domain = spec.FUNCTIONS[name]
    bad = [i for i, (lo, hi) in enumerate(spec.blocks(domain)) if format(oracle_lib.pd_digest(fid, lo, hi), "016x") != g["blocks"][i]]
    assert not bad, f"{name}: blocks {bad[:8]} differ from the reference"


@pytest.mark.parametrize("name", list(spec.FUNCTIONS))
def test_oracle_samples(name, oracle_lib, golden):
    g = golden["functions"][name]
    ins = [i for i, _ in g["samples"]]
    want = [o for _, o in g["samples"]]
    a_in = (ctypes.c_uint64 * len(ins))(*ins)
    a_out = (ctypes.c_uint32 * len(ins))()
    assert oracle_lib.pd_eval(g["id"], a_in, a_out, len(ins)) == 0
    got = list(a_out)
    diff = [(hex(i), hex(w), hex(o)) for i, w, o in zip(ins, want, got) if w != o]
    assert not diff, diff[:5]


def _eval(lib, fid, ins):
    ins = [int(x) for x in ins]
    a_in = (ctypes.c_uint64 * len(ins))(*ins)
    a_out = (ctypes.c_uint32 * len(ins))()
    assert lib.pd_eval(fid, a_in, a_out, len(ins)) == 0
    return np.array(list(a_out), dtype=np.uint64)


def test_f16_is_ieee_rounding(oracle_lib):
    """Every non-NaN f32 in a 2^20 sample rounds to numpy's float16 bits."""
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    keep = ~np.isnan(x)
    bits, x = bits[keep], x[keep]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16).astype(np.uint64)
    got = _eval(oracle_lib, spec.FUNCTIONS["f32_to_f16"][0], bits)
    assert np.array_equal(got, want)


def test_bf16_is_nearest_even(oracle_lib):
    """bf16 of an f32: the nearest of the two bf16 neighbours, ties to the even one."""
    rng = np.random.default_rng(8)
    bits = rng.integers(0, 0x7F7F0000, size=1 << 16, dtype=np.uint64).astype(np.uint32)
    got = _eval(oracle_lib, spec.FUNCTIONS["f32_to_bf16"][0], bits).astype(np.uint32)
    lo = (bits >> 16).astype(np.uint64)
    x = bits.view(np.float32).astype(np.float64)
    down = (lo << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    up = ((lo + 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    nearest = np.where(x - down < up - x, lo, np.where(x - down > up - x, lo + 1, np.where(lo % 2 == 0, lo, lo + 1)))
    assert np.array_equal(got, nearest.astype(np.uint32))


def test_libm_close_to_numpy(oracle_lib):
    """The fdlibm-method functions are within a few ulp of numpy's f64 values."""
    rng = np.random.default_rng(9)
    x = rng.uniform(-20, 20, size=1 << 14).astype(np.float32)
    bits = x.view(np.uint32)
    import math
    for name, f in (("expf", np.exp), ("tanhf", np.tanh), ("erff", np.vectorize(math.erf))):
        got = _eval(oracle_lib, spec.FUNCTIONS[name][0], bits).astype(np.uint32).view(np.float32)
        want = f(x.astype(np.float64))
        ok = np.isclose(got, want, rtol=3e-7, atol=1e-37) | (np.isinf(got) & (want > 3e38))
        assert ok.all(), (name, x[~ok][:4], got[~ok][:4], want[~ok][:4])
    xp = np.abs(x) + np.float32(1e-3)
    got = _eval(oracle_lib, spec.FUNCTIONS["logf"][0], xp.view(np.uint32)).astype(np.uint32).view(np.float32)
    assert np.allclose(got, np.log(xp.astype(np.float64)), rtol=3e-7, atol=1e-7)


def _eval_f64(lib, fid, xs):
    xs = np.asarray(xs, np.float64)
    out = np.zeros(len(xs), np.uint64)
    assert lib.pd_eval_f64(fid, xs.ctypes.data, out.ctypes.data, len(xs)) == 0
    return out


@pytest.mark.parametrize("name", list(spec.F64))
def test_oracle_f64_matches_reference(name, oracle_lib, golden):
    """The oracle's f64 function gives the reference's digest on every block
    of its argument sample (1 in 8 any bit pattern, 1 in 8 any exponent, the
    rest |x| in [1e-9, 8192]) and the reference's bits at the specials."""
    g = golden["functions_f64"][name]
    bad = [i for i, (lo, hi) in enumerate(spec.f64_blocks()) if format(oracle_lib.pd_digest(g["id"], lo, hi), "016x") != g["blocks"][i]]
    assert not bad, f"{name}: blocks {bad} differ from the reference"
    xs = np.array([int(x, 16) for x, _ in g["specials"]], np.uint64).view(np.float64)
    got = _eval_f64(oracle_lib, g["id"], xs)
    diff = [(x, w, format(int(o), "016x")) for x, (_, w), o in zip(xs, g["specials"], got) if format(int(o), "016x") != w]
    assert not diff, diff[:5]


def test_f64_libm_close_to_numpy(oracle_lib):
    """exp, log, tanh, sin, cos within 2 ulp of numpy's f64 functions (erf of
    Python's math) on arguments away from overflow."""
    import math
    rng = np.random.default_rng(11)
    x = rng.uniform(-30, 30, size=1 << 14) * 10.0 ** rng.integers(-3, 2, size=1 << 14)
    cases = (("exp", np.exp, x), ("log", np.log, np.abs(x) + 1e-300), ("tanh", np.tanh, x),
             ("erf", np.vectorize(math.erf), x), ("sin", np.sin, x * 1e3), ("cos", np.cos, x * 1e3))
    for name, f, a in cases:
        got = _eval_f64(oracle_lib, spec.F64[name], a).view(np.float64)
        want = f(a)
        ulp = np.spacing(np.maximum(np.abs(want), np.finfo(np.float64).tiny))
        err = np.abs(got - want) / ulp
        assert np.all(err <= 2), (name, a[err > 2][:4], got[err > 2][:4], want[err > 2][:4])


def test_f64_closed_forms(oracle_lib):
    """Special values the mathematics fixes."""
    import math
    ev = lambda n, xs: _eval_f64(oracle_lib, spec.F64[n], xs).view(np.float64)
    assert list(ev("exp", [0.0, -math.inf, math.inf, 1000.0, -1000.0])) == [1.0, 0.0, math.inf, math.inf, 0.0]
    assert list(ev("log", [1.0, 0.0, math.inf])) == [0.0, -math.inf, math.inf] and np.isnan(ev("log", [-1.0]))[0]
    assert list(ev("tanh", [0.0, 25.0, -25.0, math.inf])) == [0.0, 1.0, -1.0, 1.0]
    assert list(ev("erf", [0.0, 10.0, -10.0, math.inf, -math.inf])) == [0.0, 1.0, -1.0, 1.0, -1.0]
    assert list(ev("sin", [0.0, -0.0])) == [0.0, -0.0] and list(ev("cos", [0.0])) == [1.0]
    assert np.all(np.isnan(ev("sin", [math.inf, math.nan]))) and np.all(np.isnan(ev("cos", [-math.inf])))
    # Payne-Hanek: sin of 2^k pi-free multiples far out stays in [-1, 1] and
    # sin^2 + cos^2 = 1 to rounding
    big = np.array([1e22, 1e100, 1e300, 2.0 ** 1000, 1.7976931348623157e308])
    s, c = ev("sin", big), ev("cos", big)
    assert np.all(np.abs(s * s + c * c - 1) < 1e-15)
    # sin(1e22) (a classic argument-reduction test value)
    assert abs(ev("sin", [1e22])[0] - (-0.8522008497671888)) < 1e-16
