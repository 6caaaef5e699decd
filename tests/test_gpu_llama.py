"""Config 5's Llama forward (presk_amd/llama.py) on the device at the TINY
shape (grouped-query attention, two blocks): in EXACT mode every buffer of
the forward equals the oracle's byte for byte; in FAST mode (MFMA
contractions in their declared order) the logits stay within the
reassociation band.  Also the seeded device fill the full-size forward's
parameters come from."""
import numpy as np
import pytest

from presk_amd import configs, hip, llama
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
    s = llama.TINY
    out = {}
    for dt in ("f32", "bf16", "f16"):
        p, b, names = llama.build(s, dt, mode=hip.EXACT)
        out[dt] = (cpu_program.run(p, llama.host_inputs(s)), names)
    return out


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_tiny_llama_exact_bits(oracle_tiny, dt):
    s = llama.TINY
    print(f"[llama] exact {dt}", flush=True)
    p, b, names = llama.build(s, dt, mode=hip.EXACT)
    device_run(p, llama.host_inputs(s))
    env, _ = oracle_tiny[dt]
    bad = [(ln.out, ln.low.name) for ln in p.launches if p.bufs.download(ln.out).tobytes() != env[ln.out].tobytes()]
    assert not bad, f"{len(bad)} buffers differ, first: {bad[:5]}"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_tiny_llama_fast_band(oracle_tiny, dt):
    s = llama.TINY
    print(f"[llama] fast {dt}", flush=True)
    p, b, names = llama.build(s, dt, mode=hip.FAST)
    device_run(p, llama.host_inputs(s))
    assert sum(ln.compiled.kind == "gemm" for ln in p.launches) == 9 * s.L + 1   # 6 attention, 3 SwiGLU, the head
    env, _ = oracle_tiny[dt]
    got = fmt.decode(p.bufs.download(names["logits"]), dt).astype(np.float64)
    ref = fmt.decode(env[names["logits"]], dt).astype(np.float64)
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert err < {"f32": 1e-5, "bf16": 5e-2, "f16": 8e-3}[dt], err


def test_fill_normal_is_seeded_and_normal():
    hip.init(0)
    n = 1 << 20
    bufs = {}
    for ty in ("f32", "bf16"):
        b = hip.DeviceBuffer(n * (4 if ty == "f32" else 2))
        hip.check(hip.lib().presk_hip_fill_normal(b.ptr, ty.encode(), n, 12345, 0.0, 0.02, None))
        bufs[ty] = b
    again = hip.DeviceBuffer(n * 4)
    hip.check(hip.lib().presk_hip_fill_normal(again.ptr, b"f32", n, 12345, 0.0, 0.02, None))
    other = hip.DeviceBuffer(n * 4)
    hip.check(hip.lib().presk_hip_fill_normal(other.ptr, b"f32", n, 12346, 0.0, 0.02, None))
    ones = hip.DeviceBuffer(1000 * 2)
    hip.check(hip.lib().presk_hip_fill_normal(ones.ptr, b"bf16", 1000, 7, 1.0, 0.0, None))
    hip.sync()
    x = bufs["f32"].download(np.float32, n)
    assert np.array_equal(x, again.download(np.float32, n))
    assert not np.array_equal(x, other.download(np.float32, n))
    # the bf16 fill is the f32 draw rounded once to nearest even
    assert np.array_equal(bufs["bf16"].download(np.uint16, n), fmt.encode(x, "bf16"))
    assert np.all(fmt.decode(ones.download(np.uint16, 1000), "bf16") == 1.0)
    assert abs(x.mean()) < 5e-5 and abs(x.std() - 0.02) < 1e-4
    # tails of a normal: 4.6e-3 of the mass beyond 2.83 sigma, none past 6
    beyond = np.mean(np.abs(x) > 0.02 * 2.83)
    assert 3.5e-3 < beyond < 5.7e-3 and np.max(np.abs(x)) < 0.12
