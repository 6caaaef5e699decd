"""The measured configurations as whole programs on the device.

- Config 2 (the MLP block, presk_amd.configs.mlp) in bf16, f16 and e8m15
  storage: at 256 rows in EXACT mode every buffer equals the oracle's run
  of the same program byte for byte; at the full 8 192 x 768 in FAST mode
  (MFMA contractions where the storage type has them) LayerNorm's rows have
  mean 0 and variance 1 and the block's output stays within the storage
  type's band of a float64 model on a 64-row sample.
- Config 1 (Linear 4 096 x 1 024 x 1 024, f32) at its full size against the
  oracle: EXACT bit for bit, FAST within the reassociation band.
"""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import configs, hip
from tests import cpu_program, fmt
from tests.mlp_model import MEDIAN, TOL, inputs_f64, mlp_f64

pytestmark = pytest.mark.gpu


def device_run(p, host):
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    return p


@pytest.mark.parametrize("dt", ["bf16", "f16", "e8m15"])
def test_config2_exact_bits(dt):
    print(f"[config2] exact {dt} 256 rows", flush=True)
    p, host, out, _ = configs.mlp(rows=256, dtype=dt)
    p.mode = hip.EXACT
    device_run(p, host)
    env = cpu_program.run(p, host, threads=8)
    assert not env["__overflow__"]
    bad = [ln.out for ln in p.launches if p.bufs.download(ln.out).tobytes() != env[ln.out].tobytes()]
    assert not bad, f"buffers differ: {bad}"


@pytest.mark.parametrize("dt", ["bf16", "f16", "e8m15"])
def test_config2_full_fast(dt):
    print(f"[config2] fast {dt} 8192 rows", flush=True)
    rows = 8192
    p, host, out, _ = configs.mlp(rows=rows, dtype=dt)
    device_run(p, host)
    kinds = [ln.compiled.kind for ln in p.launches]
    if dt != "e8m15":
        assert kinds.count("gemm") == 2, kinds
    v = inputs_f64(host, dt)
    # LayerNorm's output over every row: mean 0, variance var/(var+eps)
    h = fmt.decode(p.bufs.download("h"), dt).astype(np.float64).reshape(rows, 768)
    var = v["x"].var(axis=1)
    assert np.abs(h.mean(axis=1)).max() < 16 * MEDIAN[dt] + 1e-6
    assert np.abs(h.var(axis=1) - var / (var + 1e-5)).max() < 64 * MEDIAN[dt] + 1e-5
    # the block's output on a sample of rows spread over the batch
    sample = np.random.default_rng(5).choice(rows, 64, replace=False)
    got = fmt.decode(p.bufs.download(out), dt).astype(np.float64).reshape(rows, 768)[sample]
    ref, _ = mlp_f64(v, sample)
    err = np.abs(got - ref) / np.abs(ref).max()
    assert err.max() < TOL[dt], err.max()
    assert np.median(err) < MEDIAN[dt], np.median(err)


@pytest.fixture(scope="module")
def linear_oracle():
    p, host, out, _ = configs.linear()
    env = cpu_program.run(p, host, threads=8, native=True)
    return host, env[out]


@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
def test_config1_full(linear_oracle, mode):
    print(f"[config1] mode {mode} 4096x1024x1024", flush=True)
    host, want = linear_oracle
    p, _, out, _ = configs.linear()
    p.mode = mode
    device_run(p, host)
    got = p.bufs.download(out)
    if mode == hip.EXACT:
        assert got.tobytes() == want.tobytes()
        return
    assert p.launches[0].compiled.kind == "gemm"
    # two f32 orders of a sum of K terms: within 2 gamma_K sum|x w| + the bias add
    x, w = host["x"].astype(np.float64), host["w"].astype(np.float64)
    K, u = 1024, 2.0 ** -24
    gam = K * u / (1 - K * u)
    bound = 2 * gam * (np.abs(x) @ np.abs(w)) + 2 * u * (np.abs(x @ w) + np.abs(host["b"]))
    err = np.abs(got.astype(np.float64) - want.astype(np.float64)).reshape(bound.shape)
    assert np.all(err <= bound)
    assert np.median(err / bound) < 1 / 64
