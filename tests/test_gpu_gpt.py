"""The course-GPT training step (presk_amd/gpt.py) end to end on the device,
at the reference's TINY constants: in EXACT mode every buffer of the step
(loss, gradients, every intermediate) equals the oracle's byte for byte, in
f32, bf16 and f64 (the f64 arm's exp/log/tanh of the double functions); in
FAST mode the loss and gradients stay within the reassociation band of the
MFMA contractions."""
import numpy as np
import pytest

from presk_amd import configs, gpt, hip
from tests import cpu_program, fmt

pytestmark = pytest.mark.gpu


def device_run(p, host):
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    return p


@pytest.fixture(scope="module")
def oracle_tiny():
    s = gpt.TINY
    out = {}
    for dt in ("f32", "bf16", "f64"):
        p, b, names = gpt.build(s, dt, train=True, mode=hip.EXACT)
        host = gpt.host_inputs(s)
        out[dt] = (cpu_program.run(p, host), names)
    return out


@pytest.mark.parametrize("dt", ["f32", "bf16", "f64"])
def test_tiny_gpt_step_exact_bits(oracle_tiny, dt):
    s = gpt.TINY
    p, b, names = gpt.build(s, dt, train=True, mode=hip.EXACT)
    host = gpt.host_inputs(s)
    device_run(p, host)
    env, _ = oracle_tiny[dt]
    bad = []
    for ln in p.launches:
        got = p.bufs.download(ln.out)
        if got.tobytes() != env[ln.out].tobytes():
            bad.append((ln.out, ln.low.name))
    assert not bad, f"{len(bad)} buffers differ, first: {bad[:5]}"


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tiny_gpt_step_fast_band(oracle_tiny, dt):
    s = gpt.TINY
    p, b, names = gpt.build(s, dt, train=True, mode=hip.FAST)
    host = gpt.host_inputs(s)
    device_run(p, host)
    env, _ = oracle_tiny[dt]
    kinds = {ln.compiled.kind for ln in p.launches}
    assert "gemm" in kinds
    loss = float(fmt.decode(p.bufs.download(names["loss"]), dt)[0])
    want = float(fmt.decode(env[names["loss"]], dt)[0])
    tol = 1e-5 if dt == "f32" else 2e-2
    assert abs(loss - want) <= tol * abs(want), (loss, want)
    floor = 1e-3 * max(np.max(np.abs(fmt.decode(env[buf], dt))) for buf in names["grads"].values())
    for name, buf in names["grads"].items():
        got = fmt.decode(p.bufs.download(buf), dt).astype(np.float64)
        ref = fmt.decode(env[buf], dt).astype(np.float64)
        scale = max(np.max(np.abs(ref)), floor)
        err = np.max(np.abs(got - ref)) / scale
        assert err < (1e-4 if dt == "f32" else 6e-2), (name, err)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tiny_gpt_step_with_dropout_exact_bits(dt):
    """the course's dropout 0.2: the masks drawn on the device from the step
    key's site keys, and every buffer of the step, equal the oracle's"""
    from presk_amd import keys
    s = gpt.TINY
    k = keys.child(keys.from_seed(5), 2)
    p, b, names = gpt.build(s, dt, train=True, mode=hip.EXACT, dropout=0.2, step_key=k)
    host = gpt.host_inputs(s)
    device_run(p, host)
    q, _, _ = gpt.build(s, dt, train=True, mode=hip.EXACT, dropout=0.2, step_key=k)
    env = cpu_program.run(q, host)
    bad = [n for n in [m[0] for m in p.masks] + [ln.out for ln in p.launches]
           if p.bufs.download(n).tobytes() != env[n].tobytes()]
    assert not bad, f"{len(bad)} buffers differ, first: {bad[:5]}"


def test_dropout_step_graph_takes_each_steps_key():
    """recorded once as a graph; the host writes the next step's site keys to
    the device and the replay draws that step's masks"""
    from presk_amd import keys
    s = gpt.TINY
    run_key = keys.from_seed(9)
    p, b, names = gpt.build(s, "f32", train=True, mode=hip.EXACT, dropout=0.2, step_key=keys.child(run_key, 0))
    host = gpt.host_inputs(s)
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.record(graph=True)
    for step in (0, 1):
        p.set_keys(gpt.site_keys(s, keys.child(run_key, step)))
        p.run()
        hip.sync()
        q, _, _ = gpt.build(s, "f32", train=True, mode=hip.EXACT, dropout=0.2, step_key=keys.child(run_key, step))
        env = cpu_program.run(q, host)
        for name in [m[0] for m in p.masks] + [names["loss"]]:
            assert p.bufs.download(name).tobytes() == env[name].tobytes(), (step, name)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tiny_gpt_step_with_adamw_exact_bits(dt):
    """the training run's step with its optimizer (adamw.step and adamw.lr,
    f32 and bf16 storage): the clipped global norm summed in f64 through the
    edge conversions, each body's fusion groups as fusion.rs forms them (one
    nest a group, f32 inside it, only its root stored: the schedule one 0-dim
    nest, m', v' and theta' one nest a leaf), every leaf's moments and
    parameters (the blocks' leaves stacked over the layers) -- every buffer
    equal to the oracle's, replayed as a graph too"""
    s = gpt.TINY
    p, b, names = gpt.build(s, dt, train=True, mode=hip.EXACT, optimizer=True)
    host = gpt.host_inputs(s)
    host.update(gpt.optimizer_inputs(s, 150, 400))
    device_run(p, host)
    # the blocks' parameters and gradients sit in their stacked leaves, no copy
    for l in range(s.L):
        w = 4 if dt == "f32" else 2
        assert p.bufs.dev[f"b{l}.wq"].ptr == p.bufs.dev["blocks.wq"].ptr + w * l * s.D * s.D
        assert p.bufs.dev[names["grads"][f"b{l}.up.b"]].ptr == p.bufs.dev["d.blocks.up.b"].ptr + w * l * 4 * s.D
    q, _, _ = gpt.build(s, dt, train=True, mode=hip.EXACT, optimizer=True)
    env = cpu_program.run(q, host)
    outs = [ln.out for ln in p.launches]
    bad = [n for n in outs if p.bufs.download(n).tobytes() != env[n].tobytes()]
    assert not bad, f"{len(bad)} buffers differ, first: {bad[:5]}"
    assert any(ln.low.dtype == "f64" for ln in p.launches)       # the f64 sums ran
    p.record(graph=True)
    p.run()
    hip.sync()
    for k, (th, m2, v2) in names["adamw"].items():
        for n in (th, m2, v2):
            assert p.bufs.download(n).tobytes() == env[n].tobytes(), (k, n)
