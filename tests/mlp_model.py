"""An independent float64 model of config 2's MLP block (examples/spec/mlp/mlp.psk
and examples/spec/layernorm/layernorm.psk): LayerNorm over `model`, Linear,
the exact gelu x * (1 + erf(x / sqrt 2)) / 2 (crates/presk-kernel/src/lower.rs:168-171),
Linear, residual add.  Written from the programs' mathematics, not from the
nests, so it pins what presk_amd.configs.mlp computes."""
import numpy as np
from scipy.special import erf

from tests import fmt


def inputs_f64(host: dict, dt: str) -> dict:
    """The host inputs as the device holds them (rounded to storage once), in f64."""
    return {k: fmt.roundtrip(np.asarray(v, np.float32), dt).astype(np.float64) for k, v in host.items()}


def mlp_f64(v: dict, rows=None):
    """(out, h) of the block over `rows` (a slice or index array) of x."""
    x = v["x"] if rows is None else v["x"][rows]
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    h = (x - mu) / np.sqrt(var + v["eps"][0]) * v["gamma"] + v["beta"]
    u = h @ v["w1"] + v["b1"]
    g = u * (1.0 + erf(u / np.sqrt(2.0))) / 2.0
    return x + (g @ v["w2"] + v["b2"]), h


# Relative to max |out|: the storage type's rounding of each intermediate
# (h, u, gelu, y, out) and of the inputs, a few units of its last place; f32
# also its sums' rounding (K up to 3 072).  Measured on the oracle at 64
# rows: f32 1.0e-6, bf16 3.5e-3, f16 5.2e-4, e8m15 1.6e-5.
TOL = {"f32": 1e-5, "bf16": 4 * 2.0 ** -8, "f16": 4 * 2.0 ** -11, "e8m15": 4 * 2.0 ** -16}
MEDIAN = {"f32": 1e-6, "bf16": 2.0 ** -8, "f16": 2.0 ** -11, "e8m15": 2.0 ** -16}
