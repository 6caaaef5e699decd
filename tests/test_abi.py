"""The C ABI without a GPU: the library loads, exports every entry point
include/presk_hip.h declares, reads every zoo kernel back to the reference's
text (the round trip that pins its parser), and builds each one's HIP code
(hiprtc cross-compiles for gfx950 without a device)."""
import os
import re

import pytest

from presk_amd import hip
from tests import zoo

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "presk_hip.h")).read()
    declared = sorted(set(re.findall(r"\b(presk_hip_[a-z0-9_]+)\s*\(", header)))
    assert declared == sorted(hip.SYMBOLS)
    L = hip.lib()
    for name in declared:
        assert hasattr(L, name), name


@pytest.mark.parametrize("case", zoo.cases(), ids=lambda c: c[0])
def test_compile_and_read_back(case):
    _, low = case
    for mode in (hip.EXACT, hip.FAST):
        c = hip.Compiled(low.text, low.dtype, low.lanes, mode)
        assert c.read_back() == low.text
        assert c.guarded == (low.dtype in ("f16", "e8m15") and low.out_kind == "real")


def test_refuses_non_native_formats():
    text = ("kernel add (%0 : f32[2], %1 : f32[2]) -> %2 : f32[2] arith bf16 product bf16 accum f32 {\n"
            "  for i0 in 0..2 {\n    %2[i0] = (%0[i0] + %1[i0])\n  }\n}\n")
    with pytest.raises(hip.HipError) as e:
        hip.Compiled(text, "f32")
    assert e.value.code == "E7005"


def test_accepts_quantised_weights():
    """Integer weights are the native backend's to compute (their scales in
    the slots after the output, crates/presk-cranelift/src/lib.rs:1619-1624),
    and this executor's too."""
    text = ("kernel dot (%0 : f32[2, 3], %1 : int8/0[3, 2]) -> %2 : f32[2, 2] {\n"
            "  for i0 in 0..2 {\n    for i1 in 0..2 {\n      %2[i0, i1] = 0\n    }\n  }\n}\n")
    c = hip.Compiled(text, "f32")
    assert c.read_back() == text and c.n_inputs == 2


def test_malformed_text_is_an_executor_error():
    with pytest.raises(hip.HipError) as e:
        hip.Compiled("kernel x (%0 : f32[2]) -> %1 : f32[2] {\n  for i0 in 0..2 {\n", "f32")
    assert e.value.code == "E10001"


def test_noalloc_refuses_before_touching_the_device():
    """presk_hip_run_noalloc's refusals are host-side: a class kernel whose
    workspace exceeds the 64 MiB scratch (here 1 024 chunk sums of 16 400
    columns, 67.2 MB), and a generic kernel with no code object loaded (no
    presk_hip_init in this process).  No pointer is read."""
    import ctypes

    from presk_amd import lower as L
    A, O = L.ax, L.Operand
    low = L.sum_to([O(A(("batch", 65536), ("model", 16400))), O(A(("model", 16400)))], "f32")
    c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    assert c.kind == "colsum"
    table = (ctypes.c_void_p * 3)(None, None, None)
    rc = hip.lib().presk_hip_run_noalloc(c.handle, table, 0, 0, None)
    assert rc == hip.ERR
    msg = hip.lib().presk_hip_last_error().decode()
    assert msg.startswith("E10001") and "67174400 bytes of scratch" in msg, msg
    if hip._initialized is not None:
        return   # a device is set up in this process: the code object would be loaded
    g = L.unary("gelu", [O(A(("batch", 4), ("model", 8)))], "f32")
    cg = hip.Compiled(g.text, "f32", g.lanes, hip.EXACT)
    assert cg.kind == "generic"
    rc = hip.lib().presk_hip_run_noalloc(cg.handle, (ctypes.c_void_p * 2)(None, None), 0, 4, None)
    assert rc == hip.ERR and "no code object loaded" in hip.lib().presk_hip_last_error().decode()


def test_graph_branches_checked_before_any_device_work():
    """presk_hip_batch_graph_branches takes 1-8 branches, and more than one is
    refused in this build (E10001), before any capture."""
    import ctypes
    L = hip.lib()
    b = ctypes.c_void_p()
    assert L.presk_hip_batch_create(ctypes.byref(b)) == hip.OK
    try:
        for n, text in ((0, "not in 1..8"), (9, "not in 1..8"), (4, "switched off")):
            assert L.presk_hip_batch_graph_branches(b, n) == hip.ERR
            msg = L.presk_hip_last_error().decode()
            assert msg.startswith("E10001") and text in msg, msg
    finally:
        L.presk_hip_batch_release(b)


def test_short_kernelfn_tables_refused_on_the_host():
    """The KernelFn table carries no length (crates/presk-cranelift/src/
    lib.rs:38-42), so the host binding checks it: a table missing an input
    (a `sum_to` given no template operand) or holding a null pointer is
    refused before any launch, instead of the plan reading its output slot
    past the table's end."""
    from presk_amd import lower as L
    A, O = L.ax, L.Operand
    low = L.sum_to([O(A(("batch", 64), ("seq", 256), ("model", 384))), O(A(("batch", 64), ("seq", 256)))], "f32")
    c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    assert c.kind == "rows" and c.n_inputs == 2 and c.order == "lanes64x4-tree"
    with pytest.raises(ValueError, match="2 inputs"):
        c.run([0x1000, 0x2000])
    with pytest.raises(ValueError, match="non-null"):
        c.run([0x1000, None, 0x3000])

    class Buf:
        ptr = 0x1000
    ex = hip.HipExec.__new__(hip.HipExec)
    ex.mode, ex._cache = hip.FAST, {}
    with pytest.raises(ValueError, match="1 input buffers for a kernel of 2 inputs"):
        ex.run(low.text, "f32", [Buf()], Buf())


def test_mfma_probe_refuses_other_types():
    """presk_hip_mfma_probe measures bf16 and f32 MFMA loops only; any other
    type (or no iterations) is E10001 before a device is needed."""
    import ctypes
    from presk_amd import hip
    ms, fl = ctypes.c_double(), ctypes.c_double()
    for ty, it in ((b"f64", 10), (b"bf16", 0)):
        rc = hip.lib().presk_hip_mfma_probe(ty, it, None, ctypes.byref(ms), ctypes.byref(fl))
        assert rc != 0 and b"E10001" in hip.lib().presk_hip_last_error()
