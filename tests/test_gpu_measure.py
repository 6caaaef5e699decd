"""`solve --measure hip` (presk_amd/measure.py): each candidate realization
of config 3's entry (the course GPT's loss, TINY) measured on the device
gives the gap the kernel interpreter's bits give -- the oracle's run of the
same program under the same realization, against the same exact reference
(an independent float64 torch forward) -- as equal floats; a narrower
realization measures a larger gap; a run whose stores overflow measures +inf."""
import math

import numpy as np
import pytest

from presk_amd import gpt, hip
from presk_amd.measure import HipMeasure, gpt_forward, leaf_gap
from presk_amd.realize import Realization
from tests import cpu_program, fmt
from tests.test_gpt_program import torch_model

pytestmark = pytest.mark.gpu


def oracle_gap(s, host, r, ref):
    p, b, names = gpt.build(s, r.default, train=False, mode=hip.EXACT, realize=r)
    env = cpu_program.run(p, host)
    if env["__overflow__"]:
        return math.inf
    ty = next(ln.low.dtype for ln in p.launches if ln.out == names["loss"])
    out = fmt.decode(env[names["loss"]], ty).astype(np.float64)
    return leaf_gap(ref, [out])


CANDIDATES = ["f32", "bf16", "f16", "@presk_amd/realizations/course_gpt_mixed.json"]


def test_device_gaps_are_the_interpreters():
    s = gpt.TINY
    host = gpt.host_inputs(s)
    ref = [np.array([torch_model(s, host)[0]])]
    m = HipMeasure(gpt_forward(s, host), host, ref)
    gaps = {}
    for spec in CANDIDATES:
        print(f"[measure] {spec}", flush=True)
        r = Realization.parse(spec)
        g = m(r)
        assert g == oracle_gap(s, host, r, ref), spec
        gaps[spec] = g
    assert 0 < gaps["f32"] < gaps["bf16"] < math.inf and gaps["f32"] < 1e-5
    assert m.runs == len(CANDIDATES)


def test_overflow_measures_infinite():
    s = gpt.TINY
    host = {k: (np.asarray(v) * 3e4 if k in ("tok", "pos") else v) for k, v in gpt.host_inputs(s).items()}
    ref = [np.array([0.0])]
    m = HipMeasure(gpt_forward(s, host), host, ref)
    assert m(Realization.parse("f16")) == math.inf
    assert m(Realization.parse("f32")) < math.inf


def test_command_line_reads_its_reference_from_a_psk_d_file(tmp_path, capsys):
    import json
    from presk_amd import measure, pskd
    s = gpt.TINY
    host = gpt.host_inputs(s)
    loss = torch_model(s, host)[0]
    ref = str(tmp_path / "loss.psk.d")
    pskd.write(ref, "ℝ[]", pskd.Layout.from_type_text("ℝ[]"), [[[loss]]])
    assert measure.main(["--shape", "tiny", "--reference", ref, "--realize", "f32", "bf16"]) == 0
    lines = [json.loads(x) for x in capsys.readouterr().out.strip().splitlines()]
    assert [x["realization"] for x in lines] == ["f32", "bf16"]
    assert lines[0]["gap"] == oracle_gap(s, host, Realization.parse("f32"), [np.array([loss])])
    assert lines[1]["gap"] > lines[0]["gap"] and lines[0]["reference_max"] == abs(loss)
