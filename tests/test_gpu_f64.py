"""The f64 functions through the generic printer on the device: an f64 nest
applying exp, log, tanh, erf, sin or cos to every special argument of
tests/golden/spec.py (branch points, thresholds, multiples of pi/2, signed
zeros, infinities, NaNs) gives the reference's bits (tests/golden/digests.json,
from the reference's compiled presk_libm.c), and on 2^16 more arguments the
oracle's (oracle/libm.c, pinned to the same reference)."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from tests.golden import spec

pytestmark = pytest.mark.gpu


def run_unary(op, xs, mode):
    """`%1[i] = op(%0[i])` over f64 (erf is no primitive of its own, only
    inside gelu, so the nest is written as text from exp's)."""
    low = L.unary("exp", [L.Operand(L.ax(("batch", len(xs))))], "f64")
    text = low.text.replace("kernel exp", f"kernel {op}").replace("= exp(", f"= {op}(")
    c = hip.Compiled(text, "f64", low.lanes, mode)
    bx = hip.DeviceBuffer.of(np.ascontiguousarray(xs, np.float64))
    out = hip.DeviceBuffer(8 * len(xs))
    out.upload(np.full(8 * len(xs), 0xFF, np.uint8))
    c.run([bx.ptr, out.ptr])
    hip.sync()
    return text, low.lanes, out.download(np.float64)


@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
@pytest.mark.parametrize("name", list(spec.F64))
def test_f64_function_specials_and_sample(name, mode, golden):
    hip.init(0)
    g = golden["functions_f64"][name]
    xs = np.array([int(x, 16) for x, _ in g["specials"]], np.uint64).view(np.float64)
    want = np.array([int(y, 16) for _, y in g["specials"]], np.uint64)
    print(f"[f64] {name} mode {mode}: {len(xs)} specials", flush=True)
    _, _, got = run_unary(name, xs, mode)
    bad = np.nonzero(got.view(np.uint64) != want)[0]
    assert bad.size == 0, [(xs[i], hex(int(want[i])), hex(int(got.view(np.uint64)[i]))) for i in bad[:5]]
    rng = np.random.default_rng(spec.F64[name])
    sample = rng.standard_normal(1 << 16) * 10.0 ** rng.integers(-8, 4, size=1 << 16)
    if name == "log":
        sample = np.abs(sample)
    text, lanes, got = run_unary(name, sample, mode)
    ref, _ = cexec.run(text, "f64", [sample], lanes=lanes)
    assert got.tobytes() == ref.tobytes()
