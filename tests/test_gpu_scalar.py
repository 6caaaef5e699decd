"""The device's conversions and transcendentals over their whole domains:
every f32 input of expf/logf/tanhf/erff and the narrowings, every code of the
widenings, the f64 sample of the narrowings from f64, and the f64 functions
over their argument sample of 2^24.  Each block's digest must equal the
reference's (tests/golden/digests.json, made from the reference's compiled
presk_rt.h/presk_libm.c)."""
import ctypes

import pytest

from presk_amd import hip
from tests.golden import spec

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", list(spec.FUNCTIONS))
def test_device_function_everywhere(name, golden):
    hip.init(0)
    g = golden["functions"][name]
    fid, domain = spec.FUNCTIONS[name]
    bad = []
    for i, (lo, hi) in enumerate(spec.blocks(domain)):
        d = ctypes.c_uint64()
        hip.check(hip.lib().presk_hip_scalar_digest(fid, lo, hi, ctypes.byref(d)))
        if format(d.value, "016x") != g["blocks"][i]:
            bad.append(i)
    print(f"[scalar] {name}: {len(bad)} of {len(spec.blocks(domain))} blocks differ", flush=True)
    assert not bad, f"{name}: blocks {bad[:8]} differ from the reference"


def test_expf_fast_path_is_expf(golden):
    """the softmax's exp on (-87.34, 0] (pk_expf_le0, taken where
    pk_expf_le0_ok holds, pk_expf elsewhere) has expf's digest over every f32"""
    hip.init(0)
    g = golden["functions"]["expf"]
    _, domain = spec.FUNCTIONS["expf"]
    bad = []
    for i, (lo, hi) in enumerate(spec.blocks(domain)):
        d = ctypes.c_uint64()
        hip.check(hip.lib().presk_hip_scalar_digest(6, lo, hi, ctypes.byref(d)))
        if format(d.value, "016x") != g["blocks"][i]:
            bad.append(i)
    assert not bad, f"blocks {bad[:8]} differ from the reference's expf"


def test_softmax_quotient_is_the_division():
    """the softmax's quotient x / z (Markstein's correction step with 1/z
    where pk_div_by_ok says it is exact, the division elsewhere) equals the
    correctly rounded f32 division over every f32 x, each against one of 16
    divisors from 1 to 2^24 (in 2^32 / 2^28 blocks, digest against digest)"""
    hip.init(0)
    step = 1 << 28
    for lo in range(0, 1 << 32, step):
        a, b = ctypes.c_uint64(), ctypes.c_uint64()
        hip.check(hip.lib().presk_hip_scalar_digest(7, lo, lo + step, ctypes.byref(a)))
        hip.check(hip.lib().presk_hip_scalar_digest(8, lo, lo + step, ctypes.byref(b)))
        assert a.value == b.value, hex(lo)


@pytest.mark.parametrize("k", range(8))
def test_division_by_a_constant_is_the_division(k):
    """the printed nests' division by a constant, pk_div_rc (the f64 product
    with RN64(1/c), rounded to f32), equals the correctly rounded division
    for every f32 dividend, for each of eight divisors (selftest.hip's
    scan_divisor: sqrt 2, sqrt(2 pi), 3, 0.1, 2 - 2^-23, a subnormal,
    3e30, -6)"""
    hip.init(0)
    d = ctypes.c_uint64()
    hip.check(hip.lib().presk_hip_scalar_digest(70 + k, 0, 1 << 32, ctypes.byref(d)))
    print(f"[div] divisor {k}: {d.value} of 2^32 dividends differ", flush=True)
    assert d.value == 0, d.value


@pytest.mark.parametrize("name", list(spec.F64))
def test_device_f64_function_sample(name, golden):
    hip.init(0)
    g = golden["functions_f64"][name]
    bad = []
    for i, (lo, hi) in enumerate(spec.f64_blocks()):
        d = ctypes.c_uint64()
        hip.check(hip.lib().presk_hip_scalar_digest(g["id"], lo, hi, ctypes.byref(d)))
        if format(d.value, "016x") != g["blocks"][i]:
            bad.append(i)
    print(f"[scalar] {name} (f64): {len(bad)} of 16 blocks differ", flush=True)
    assert not bad, f"{name}: blocks {bad} differ from the reference"
