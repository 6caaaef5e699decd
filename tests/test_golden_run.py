"""The golden entries on the CPU: the oracle's run of each program
(tests/golden/run_entries.py) against the reference's exact outputs
(tests/golden/run/*.snap) within the storage type's conformance band, and
the inputs' synthesis against the snapshots it feeds -- three independent
snapshots (LayerNorm, RMSNorm, the MLP's loss) agree with float64 models of
the drawn inputs to 1e-11, which pins Key::from_seed / split, the
Box-Muller normals and xavier_uniform's draws (tests/golden/make_run.py)."""
import numpy as np
import pytest
from scipy.special import erf

from tests import cpu_program
from tests.golden import run_entries as R


def test_drawn_inputs_reproduce_the_snapshots_in_f64():
    v = R.inputs()
    x = v["norm.x"]
    mu = x.mean(1, keepdims=True)
    ln = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    rms = x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-6)
    assert np.allclose(ln.ravel(), R.snapshot("layernorm_apply"), rtol=1e-11, atol=1e-12)
    assert np.allclose(rms.ravel(), R.snapshot("rmsnorm_apply"), rtol=1e-11, atol=1e-12)
    u = v["mlp.x"] @ v["mlp.w1"]
    yh = (u * (1 + erf(u / np.sqrt(2))) / 2) @ v["mlp.w2"]
    assert abs(((yh - v["mlp.y"]) ** 2).mean() - R.snapshot("mlp_mse")[0]) < 1e-11


def _oracle(p, host):
    return cpu_program.run(p, host)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("entry", ["layernorm_apply", "rmsnorm_apply"])
def test_norms(entry, dt):
    p, host, out = (R.layernorm if entry == "layernorm_apply" else R.rmsnorm)(dt)
    env = _oracle(p, host)
    from tests import fmt
    got = fmt.decode(env[out], dt)
    assert np.all(R.within(got, R.snapshot(entry), dt))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_mlp_mse_and_grad(dt):
    from tests import fmt
    p, host, names = R.mlp(dt, grad=True)
    env = _oracle(p, host)
    assert np.all(R.within(fmt.decode(env[names["mse"]] if "mse" in names else env["mse"], dt), R.snapshot("mlp_mse"), dt))
    want = R.snapshot("mlp_mse_grad")
    for leaf in ("l1.w", "l1.b", "l2.w", "l2.b"):
        ok = R.within(fmt.decode(env[names[leaf]], dt), want[leaf], dt)
        assert np.all(ok), (leaf, np.flatnonzero(~ok)[:5])


def test_minigpt_zero_head():
    from tests import fmt
    p, host, names = R.minigpt("f32")
    env = _oracle(p, host)
    logits = fmt.decode(env[names["logits"]], "f32")
    assert np.all(logits == 0.0) and R.snapshot("minigpt_forward").size == logits.size
    assert np.all(R.within(env[names["loss"]], R.snapshot("minigpt_loss"), "f32"))
