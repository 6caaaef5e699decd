"""The oracle's conversions and libm against the reference's own C runtime.

tests/golden/digests.json holds, per function, the digest of every block of
its domain computed from crates/presk-export-c/c/presk_rt.h and presk_libm.c
(tests/golden/make_golden.py).  Every block of the oracle's restatement must
give the same digest: every f32 input for expf/logf/tanhf/erff and the
narrowings, every code for the widenings.  Independent checks beside the
reference's: numpy's IEEE binary16 rounding, and closed forms.
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
