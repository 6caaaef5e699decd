"""The device's conversions and transcendentals over their whole domains:
every f32 input of expf/logf/tanhf/erff and the narrowings, every code of the
widenings, the f64 sample of the narrowings from f64.  Each block's digest
must equal the reference's (tests/golden/digests.json, made from the
reference's compiled presk_rt.h/presk_libm.c)."""
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
