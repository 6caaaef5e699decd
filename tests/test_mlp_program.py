"""Config 2's program (presk_amd.configs.mlp: LayerNorm's nests, Linear's
`dot+add`, gelu, Linear, residual `add`) run by the oracle, against an
independent float64 model of the block, in every storage type.  A dropped
bias, a transposed weight or a wrong normalisation fails the f16, e8m15 or
f32 band by orders of magnitude."""
import numpy as np
import pytest

from presk_amd import configs
from tests import cpu_program, fmt
from tests.mlp_model import MEDIAN, TOL, inputs_f64, mlp_f64


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16", "e8m15"])
def test_mlp_program_matches_f64_model(dt):
    rows = 48
    p, host, out, flops = configs.mlp(rows=rows, dtype=dt)
    assert flops == 2 * 2 * rows * 768 * 3072
    env = cpu_program.run(p, host, threads=8)
    assert not env["__overflow__"]
    got = fmt.decode(env[out], dt).astype(np.float64).reshape(rows, 768)
    ref, h = mlp_f64(inputs_f64(host, dt))
    scale = np.abs(ref).max()
    err = np.abs(got - ref) / scale
    assert err.max() < TOL[dt], err.max()
    assert np.median(err) < MEDIAN[dt], np.median(err)
    # the LayerNorm output itself (gamma 1, beta 0): rows of mean 0, variance 1
    hh = fmt.decode(env["h"], dt).astype(np.float64).reshape(rows, 768)
    assert np.abs(hh - h).max() < 8 * TOL[dt] * np.abs(h).max()
