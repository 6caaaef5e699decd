"""Integer weights (BufKind::Quant) on the device against the oracle, bit for
bit: a contraction reading int8 or int4 weights with one f32 scale per
channel, the stored axis kept by the kernel's view or split into two axes
(span 2), scalar loads and the tiled layout's vector loads (f32, 4 lanes),
in every storage type's arithmetic: EXACT through the generic printer's
loads, bit for bit; FAST on the f32 MFMA kernel from the weights' loads
(f32(q) * s into an f32 copy, the other operand widened exactly, the f32
sums stored into the storage type afterwards with the epilogue), within the
band of two f32 orders of the same sums.  The scales ride in the slot after the output, the
overflow flag after them (crates/presk-cranelift/src/lib.rs:1609-1629)."""
import ctypes

import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from presk_amd import quant as Q
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand


def case(bits, span, dt, J):
    rng = np.random.default_rng(bits * 10 + span + J)
    K = 64
    w = rng.standard_normal((K, J))
    qt = Q.quantize(w, (K, J), Q.Quant(bits, 0))
    x = rng.standard_normal((50, K)).astype(np.float32)
    if span == 1:
        low = L.dot([O(A(("batch", 50), K)), O(A(K, J))], dt)
        kind = Q.of_quant(qt, (K, J))
    else:
        low = L.ein([O(A(("batch", 50), ("a", 4), ("b", 16))), O(A(("a", 4), ("b", 16), ("out", J)))],
                    [["batch", "a", "b"], ["a", "b", "out"]], ["batch", "out"], dt)
        kind = Q.of_quant(qt, (4, 16, J))
    return Q.mark(low.text, 1, kind), low, fmt.encode(x, dt), qt


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16", "e8m15"])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("span,J", [(1, 3), (1, 8), (2, 8)])
@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
def test_integer_weights_exact(dt, bits, span, J, mode):
    text, low, x, qt = case(bits, span, dt, J)
    print(f"[quant] {dt} int{bits} span {span} J {J} mode {mode} lanes {low.lanes}", flush=True)
    want, flag = cexec.run(text, dt, [x, (qt.data, qt.scales)], lanes=low.lanes)
    c = hip.Compiled(text, dt, low.lanes, mode)
    assert c.kind == ("generic" if mode == hip.EXACT else "gemm"), c.kind
    bx, bq, bs = hip.DeviceBuffer.of(x), hip.DeviceBuffer.of(qt.data), hip.DeviceBuffer.of(qt.scales)
    out = hip.DeviceBuffer(want.nbytes)
    out.upload(np.full(want.nbytes, 0xFF, np.uint8))
    f = hip.DeviceBuffer(4)
    f.zero()
    ptrs = [bx.ptr, bq.ptr, out.ptr, bs.ptr] + ([f.ptr] if c.guarded else [])
    c.run(ptrs)
    hip.sync()
    got = out.download(want.dtype)
    if c.guarded:
        assert bool(f.download(np.uint32, 1)[0]) == flag
    if mode == hip.EXACT:
        assert got.tobytes() == want.tobytes()
        return
    assert c.order == "mfma-f32-k4", c.order
    # two f32 orders of the same K products of the loads: 2 gamma_K S, plus
    # one unit of the storage type for the sum and the result
    xs = fmt.decode(x, dt).astype(np.float64).reshape(50, -1)
    wv = qt.dequantize().astype(np.float64).reshape(xs.shape[1], -1)
    K = xs.shape[1]
    S = np.abs(xs) @ np.abs(wv)
    g = fmt.decode(got, dt).astype(np.float64).reshape(S.shape)
    r = fmt.decode(want, dt).astype(np.float64).reshape(S.shape)
    unit = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10, "e8m15": 2.0 ** -15}[dt]
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    bound = 2 * gamma * S + unit * (S + 2 * np.maximum(np.abs(r), np.abs(g))) + 1e-30
    assert np.all(np.abs(g - r) <= bound), np.max(np.abs(g - r) / bound)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("mode", [hip.EXACT, hip.FAST])
def test_quantised_llama_exact(dt, mode):
    """Config 5's program at TINY with the realization's `quant` map (int8
    attention projections, the output projection read through a split view,
    int4 down projections, a pow2 head): every buffer equals the oracle's."""
    from presk_amd import configs, llama
    from presk_amd.realize import Realization
    from tests import cpu_program
    from tests.test_quant import QUANT_LLAMA
    print(f"[quant] llama {dt} mode {mode}", flush=True)
    s = llama.TINY
    r = Realization.of_json({"default": dt, "order": {"kind": "sequential"}, "quant": QUANT_LLAMA})
    p, _, names = llama.build(s, dt, mode=mode, realize=r)
    host = llama.host_inputs(s)
    env = cpu_program.run(p, host)
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    if mode == hip.EXACT:
        bad = [ln.out for ln in p.launches if p.bufs.download(ln.out).tobytes() != env[ln.out].tobytes()]
        assert not bad, bad[:5]
    else:
        got = fmt.decode(p.bufs.download(names["logits"]), dt).astype(np.float64)
        ref = fmt.decode(env[names["logits"]], dt).astype(np.float64)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < (1e-5 if dt == "f32" else 5e-2)
