"""The host's f64 -> storage conversion (presk_amd.configs.encode64, the
reference's `Buf::of`, crates/presk-rt/src/lib.rs:868-876) against the
oracle's restatement (`po_convert`, itself pinned against the reference's
runtime presk_convert in tests/test_oracle_convert.py): f32 rounded once,
bf16 through the f32, binary16 and e8m15 rounded once from the f64 -- on
samples over every binade, ties, subnormals, overflow, infinities, NaNs."""
import numpy as np
import pytest

from presk_amd import configs
from tests import cpu_program


def samples():
    rng = np.random.default_rng(3)
    e = rng.integers(-160, 140, 200_000)
    x = rng.standard_normal(200_000) * np.exp2(e.astype(np.float64))
    # ties and neighbours of ties at the storage widths: values with few bits
    m = rng.integers(1, 1 << 17, 50_000).astype(np.float64)
    ties = np.concatenate([m * 2.0 ** rng.integers(-40, 20, m.size), (m + 0.5) * 2.0 ** -17 * 2.0 ** rng.integers(-30, 16, m.size)])
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 65504.0, 65519.999, 65520.0, 6e-8, 5.96e-8, 2.98e-8,
                        3.4e38, 3.4028e38, 3.40282347e38, 1e-45, 1e-38, 1.1754943508222875e-38, 2.0 ** -149, 2.0 ** -150,
                        5e-324, 2.2250738585072014e-308, 1.7976931348623157e308])
    return np.concatenate([x, -x[:1000], ties, special])


@pytest.mark.parametrize("ty", ["f32", "bf16", "f16", "e8m15"])
def test_encode64_is_buf_of(ty):
    x = samples()
    got = configs.encode64(x, ty)
    want, _ = cpu_program.convert(x, "f64", ty, x.size)
    assert got.tobytes() == np.ascontiguousarray(want).tobytes()
