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


def test_refuses_quantised_weights():
    text = ("kernel dot (%0 : f32[2, 3], %1 : int8/0[3, 2]) -> %2 : f32[2, 2] {\n"
            "  for i0 in 0..2 {\n    for i1 in 0..2 {\n      %2[i0, i1] = 0\n    }\n  }\n}\n")
    with pytest.raises(hip.HipError) as e:
        hip.Compiled(text, "f32")
    assert e.value.code == "E7005"


def test_malformed_text_is_an_executor_error():
    with pytest.raises(hip.HipError) as e:
        hip.Compiled("kernel x (%0 : f32[2]) -> %1 : f32[2] {\n  for i0 in 0..2 {\n", "f32")
    assert e.value.code == "E10001"
