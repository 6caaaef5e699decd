"""The reference's golden entries on the device (tests/golden/run_entries.py):
LayerNorm{8}.apply, RMSNorm{8}.apply, the MLP's mse and every parameter's
gradient (mse_grad), and the MiniGPT forward and loss with its zero head,
each compared with the reference's exact output (the MPFR interpreter at 256
bits, tests/golden/run/*.snap) within the storage type's conformance band
(crates/presk-kernel/tests/conformance.rs:53-69), in EXACT mode (also
byte-equal to the oracle's run) and in FAST mode."""
import numpy as np
import pytest

from presk_amd import configs, hip
from tests import cpu_program, fmt
from tests.golden import run_entries as R

pytestmark = pytest.mark.gpu


def device(p, host):
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    return p


def read(p, name, dt):
    return fmt.decode(p.bufs.download(name), dt).astype(np.float64)


@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("entry", ["layernorm_apply", "rmsnorm_apply", "mlp_mse_grad"])
def test_golden_entry(entry, dt, mode):
    print(f"[golden] {entry} {dt} mode {mode}", flush=True)
    if entry == "mlp_mse_grad":
        p, host, names = R.mlp(dt, grad=True, mode=mode)
    else:
        p, host, out = (R.layernorm if entry == "layernorm_apply" else R.rmsnorm)(dt, mode=mode)
        names = {"out": out}
    device(p, host)
    if mode == hip.EXACT:
        env = cpu_program.run(p, host)
        bad = [ln.out for ln in p.launches if p.bufs.download(ln.out).tobytes() != np.ascontiguousarray(env[ln.out]).tobytes()]
        assert not bad, bad[:5]
    if entry == "mlp_mse_grad":
        assert np.all(R.within(read(p, "mse", dt), R.snapshot("mlp_mse"), dt))
        want = R.snapshot("mlp_mse_grad")
        for leaf in ("l1.w", "l1.b", "l2.w", "l2.b"):
            assert np.all(R.within(read(p, names[leaf], dt), want[leaf], dt)), leaf
    else:
        assert np.all(R.within(read(p, names["out"], dt), R.snapshot(entry), dt))


@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
def test_golden_minigpt_zero_head(mode):
    print(f"[golden] minigpt mode {mode}", flush=True)
    p, host, names = R.minigpt("f32", mode=mode)
    device(p, host)
    logits = read(p, names["logits"], "f32")
    assert logits.size == R.snapshot("minigpt_forward").size and np.all(logits == 0.0)
    assert np.all(R.within(read(p, names["loss"], "f32"), R.snapshot("minigpt_loss"), "f32"))
