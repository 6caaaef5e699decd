"""presk_hip_run_noalloc: the KernelFn call that allocates nothing, its
kernels' workspaces (split-K partials, chunk sums, mask bits) in the
library's fixed scratch array, against presk_hip_run (its own workspaces)
through the C ABI, bit for bit.  Two calls in a row on each class, the
second with a smaller input, so the second reads scratch the first left
behind."""
import ctypes

import numpy as np
import pytest

from presk_amd import hip
from presk_amd import lower as L
from tests import zoo

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand


def pairs():
    """(name, mode, kind, big, small) kernels of one class."""
    def vjp_r(dt, t):
        return L.dot_vjp_r([O(A(("batch", 4), ("seq", t), 96)), O(A(("batch", 4), ("seq", t), 80))], dt)

    def masked(dt, t):
        s = O(A(("batch", 3), ("heads", 2), ("seq", t), ("seq2", t)))
        return L.masked_softmax("seq2", [s, O(A(("seq", t), ("seq2", t)), "idx")], dt)

    def colsum(dt, t):
        return L.sum_to([O(A(("batch", 7), ("seq", t), ("model", 96))), O(A(("model", 96)))], dt)

    def gelu(dt, t):
        return L.unary("gelu", [O(A(("batch", 7), ("seq", t), ("model", 96)))], dt)

    out = []
    for dt in ("f32", "bf16"):
        out.append((f"dot_vjp_r-split-{dt}", hip.FAST, "gemm", vjp_r(dt, 1200), vjp_r(dt, 600)))
        out.append((f"masked_softmax_long-{dt}", hip.EXACT, "rows", masked(dt, 400), masked(dt, 300)))
        out.append((f"sum_to-{dt}", hip.FAST, "colsum", colsum(dt, 600), colsum(dt, 300)))
        out.append((f"gelu-{dt}", hip.EXACT, "generic", gelu(dt, 60), gelu(dt, 30)))
    # e8m15: the operands' and the output's f32 widenings, then the split-K
    # partials, at 256-byte-aligned offsets of the same scratch
    out.append(("dot_vjp_r-split-e8m15", hip.FAST, "gemm", vjp_r("e8m15", 1200), vjp_r("e8m15", 600)))
    return out


def _launch(fn, c, low, seed):
    ins = [hip.DeviceBuffer.of(a) for a in zoo.inputs(low, seed=seed)]
    n = 1
    for a in low.out_axes:
        n *= a.len
    out = hip.DeviceBuffer(max(n, 1) * hip.STORAGE_BYTES[low.dtype])
    out.upload(np.full(out.nbytes, 0xFF, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    ptrs = [b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else [])
    table = (ctypes.c_void_p * len(ptrs))(*ptrs)
    hip.check(fn(c.handle, table, 0, max(c.split_bound, 0), None))
    hip.sync()
    return out.download(np.uint8), ins


@pytest.mark.parametrize("case", pairs(), ids=lambda c: c[0])
def test_noalloc_equals_run(case):
    name, mode, kind, big, small = case
    print(f"[noalloc] {name}", flush=True)
    ex = hip.HipExec(0, mode=mode)
    lib = hip.lib()
    cb = ex.compiled(big.text, big.dtype, big.lanes)
    cs = ex.compiled(small.text, small.dtype, small.lanes)
    assert cb.kind == kind and cs.kind == kind
    if kind == "gemm":
        assert "-split" in cb.order and "-split" in cs.order, (cb.order, cs.order)
    want_b, _ = _launch(lib.presk_hip_run, cb, big, 1)
    want_s, _ = _launch(lib.presk_hip_run, cs, small, 2)
    got_b, _ = _launch(lib.presk_hip_run_noalloc, cb, big, 1)
    got_s, _ = _launch(lib.presk_hip_run_noalloc, cs, small, 2)
    assert got_b.tobytes() == want_b.tobytes()
    assert got_s.tobytes() == want_s.tobytes()
