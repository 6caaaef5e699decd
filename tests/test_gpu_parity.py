"""Bit parity of the device with the oracle on every zoo nest (EXACT mode:
every sum in index order, `ReductionOrder::Sequential`).

For each nest: seeded inputs in its storage type, the oracle's output
(oracle/cexec.py, the kernel interpreter's native semantics) and the
executor's, byte for byte, and the overflow flag.  The device output buffer
starts as 0xff bytes, so an element the kernel never writes shows up."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from tests import zoo

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ex():
    return hip.HipExec(0, mode=hip.EXACT)


def run_device(ex, low, ins):
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    bufs = [hip.DeviceBuffer.of(a) for a in ins]
    out_ty = k.output.ty
    nbytes = k.output.numel * hip.STORAGE_BYTES[out_ty]
    out = hip.DeviceBuffer(nbytes)
    out.upload(np.full(max(nbytes, 1), 0xFF, dtype=np.uint8))
    try:
        ex.run(low.text, low.dtype, bufs, out, lanes=low.lanes)
        flag = False
    except hip.HipError as e:
        if e.code != "E7007":
            raise
        flag = True
    return out.download(np.uint8, nbytes), flag


@pytest.mark.parametrize("case", zoo.cases(), ids=lambda c: c[0])
def test_exact_bits(ex, case):
    name, low = case
    print(f"[parity] {name}", flush=True)
    ins = zoo.inputs(low, seed=1)
    want, want_flag = cexec.run(low.text, low.dtype, ins, lanes=low.lanes)
    got, got_flag = run_device(ex, low, ins)
    assert got_flag == want_flag
    w = want.view(np.uint8)
    assert got.tobytes() == w.tobytes(), f"{name}: {np.count_nonzero(got != w)} bytes differ"


@pytest.mark.parametrize("dt", ["f16", "e8m15"])
def test_overflow_guard(ex, dt):
    """A store that turns a finite value into an infinity raises E7007
    (crates/presk-rt/src/codes.rs:120-136); the largest finite values do not."""
    from presk_amd import lower as L
    from tests import fmt
    x = L.Operand(L.ax(("batch", 4), 8))
    low = L.elementwise_binary("add", [x, x], dt)
    if dt == "f16":
        a, b = np.float32(60000.0), np.float32(6000.0)          # 66000 >= 65520
    else:
        a = np.uint32(0x7F7FFF00).view(np.float32)              # the largest finite e8m15
        b = np.float32(2.0 ** 111)                              # sum = (2 - 2^-16) 2^127, the threshold
    ins = [fmt.encode(np.full((4, 8), a, np.float32), dt), fmt.encode(np.full((4, 8), b, np.float32), dt)]
    _, flag = cexec.run(low.text, dt, ins)
    assert flag
    with pytest.raises(hip.HipError) as e:
        ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], hip.DeviceBuffer(4 * 8 * hip.STORAGE_BYTES[dt]))
    assert e.value.code == "E7007"
    small = np.full((4, 8), 2.0, dtype=np.float32)
    ins = [fmt.encode(small, dt), fmt.encode(small, dt)]
    _, flag = cexec.run(low.text, dt, ins)
    assert not flag
    ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], hip.DeviceBuffer(4 * 8 * hip.STORAGE_BYTES[dt]))


def _wide_cases():
    """Elementwise nests of 2 048 x 512 (a million iterations: the printer's
    16-byte form, each thread VEC consecutive outputs; smaller nests keep a
    thread an iteration): a unary, a broadcast binary and the LayerNorm tail's
    six-step chain."""
    from presk_amd import lower as L
    A, O = L.ax, L.Operand
    x = O(A(("batch", 8), ("seq", 256), ("model", 512)))
    r = O(A(("batch", 8), ("seq", 256)))
    b = O(A(("model", 512)))
    for dt in ("f32", "bf16", "f16"):
        yield f"gelu-{dt}", L.unary("gelu", [x], dt)
        yield f"sub-{dt}", L.elementwise_binary("sub", [x, r], dt)
        yield f"layernorm_tail-{dt}", L.fused(
            [("sub", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("in", 3)]), ("sqrt", [("step", 1)]),
             ("div", [("step", 0), ("step", 2)]), ("mul", [("step", 3), ("in", 4)]), ("add", [("step", 4), ("in", 5)])],
            [x, r, r, O([]), b, b], x.axes, dt)


@pytest.mark.parametrize("case", list(_wide_cases()), ids=lambda c: c[0])
def test_exact_bits_vectorized(ex, case):
    name, low = case
    print(f"[parity] wide {name}", flush=True)
    ins = zoo.inputs(low, seed=4)
    want, want_flag = cexec.run(low.text, low.dtype, ins, lanes=low.lanes, threads=8)
    got, got_flag = run_device(ex, low, ins)
    assert got_flag == want_flag
    w = want.view(np.uint8)
    assert got.tobytes() == w.tobytes(), f"{name}: {np.count_nonzero(got != w)} bytes differ"
