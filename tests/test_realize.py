"""The realization file: the reference's schema and precedence
(crates/presk-rt/src/lib.rs:370-455) -- a site's own type, else its
function's, else the default; parameters at rest; the fields this executor
does not compute refused with E7005.  The reference's own fixtures parse."""
import json
import os

import pytest

from presk_amd.realize import Realization

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_precedence():
    r = Realization.of_json({"default": "f32", "order": {"kind": "sequential"},
                             "storage": {"MLP.apply/u": "f16"}, "functions": {"MLP.apply": "bf16"},
                             "params": {"head": "bf16"}})
    assert r.dtype_at("MLP.apply/u") == "f16"
    assert r.dtype_at("MLP.apply/g") == "bf16"
    assert r.dtype_at("LayerNorm.apply/mu") == "f32"
    assert r.param_dtype("head") == "bf16" and r.param_dtype("tok") == "f32"
    assert Realization.parse("bf16").dtype_at("x/y") == "bf16"


def test_refusals():
    for field in ("arith", "product", "accum", "scaled"):
        with pytest.raises(ValueError, match="E7005"):
            Realization.of_json({"default": "f32", "order": {"kind": "sequential"}, field: {"a/b": "f32"}})
    with pytest.raises(ValueError, match="E7005"):
        Realization.of_json({"default": "int8", "order": {"kind": "sequential"}})


def test_authored_file_parses():
    r = Realization.parse("@" + os.path.join(ROOT, "presk_amd", "realizations", "course_gpt_mixed.json"))
    assert r.dtype_at("SelfAttention.apply/probs") == "f32"
    assert r.dtype_at("MLP.apply/u") == "bf16"


# the reference's own realization fixtures (examples/tests/plan/*.json), as
# data: their storage and params maps, read with the same schema
FIXTURE = {"default": "f16", "order": {"kind": "sequential"},
           "storage": {"Embedding.apply/%7": "f32", "LayerNorm.apply/%10": "bf16", "SelfAttention.apply/%14": "f32",
                       "MLP.apply/%4": "e8m15", "MiniGPT.apply/%11": "f32"},
           "params": {"head": "e8m15", "blocks.mlp.l2.w": "bf16"}}


def test_reference_fixture_schema():
    r = Realization.of_json(json.loads(json.dumps(FIXTURE)))
    assert r.dtype_at("MLP.apply/%4") == "e8m15"
    assert r.dtype_at("MLP.apply/%5") == "f16"
    assert r.param_dtype("head") == "e8m15"
