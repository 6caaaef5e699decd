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


@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("entry", ["rope_attention2", "rope_attention3", "concat_loss_grad", "stack_grad",
                                   "minigpt_next_token"])
def test_newer_golden_entry(entry, dt, mode):
    """Attention with RoPE (slices, concat, sin/cos, the masked softmax, the
    projections' `ein`s), the concat toy's loss and gradient (slices of index
    and real tensors, `slice_vjp`, min/max/clamp and their adjoints,
    `embed_vjp`), the stacked fold's gradient, and next_token's `index` and
    scale (the draw on the host): each within the conformance band of the
    reference's exact output, and in EXACT mode byte-equal to the oracle."""
    print(f"[golden] {entry} {dt} mode {mode}", flush=True)
    if entry.startswith("rope"):
        p, host, names = R.rope_attention(dt, int(entry[-1]), mode=mode)
    elif entry == "concat_loss_grad":
        p, host, names = R.concat_toy(dt, grad=True, mode=mode)
    elif entry == "stack_grad":
        p, host, names = R.stack_tower(dt, mode=mode)
    else:
        p, host, names = R.next_token(dt, mode=mode)
    device(p, host)
    if mode == hip.EXACT:
        env = cpu_program.run(p, host)
        bad = [ln.out for ln in p.launches if p.bufs.download(ln.out).tobytes() != np.ascontiguousarray(env[ln.out]).tobytes()]
        assert not bad, bad[:5]
    if entry.startswith("rope"):
        assert np.all(R.within(read(p, names["out"], dt), R.snapshot(entry), dt))
    elif entry == "concat_loss_grad":
        assert np.all(R.within(read(p, names["loss"], dt), R.snapshot("concat_loss"), dt))
        want = R.snapshot(entry)
        for leaf in ("tok", "head", "qkv.wq", "qkv.wk", "qkv.wv"):
            assert np.all(R.within(read(p, names[leaf], dt), want[leaf], dt)), leaf
    elif entry == "stack_grad":
        want = R.snapshot(entry)
        for leaf in ("blocks.w", "blocks.b"):
            got = np.concatenate([read(p, n, dt).ravel() for n in names[leaf]])
            assert np.all(R.within(got, want[leaf], dt)), leaf
    else:
        scaled = read(p, names["scaled"], dt).reshape(2, 64)
        assert np.array_equal(R.sample_rows(scaled, R.inputs()["next.u"]), R.snapshot(entry))
