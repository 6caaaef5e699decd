"""The lowering restatement (presk_amd/lower.py) against more of the
reference's own kernel texts: the kernels its `presk explain` documents print
for LayerNorm{8} (batch 3), MLP{4, 16} (batch 2, a bf16 bias, an f64 loss),
the tutorial's model in f32, under its typed realization (f64 with f32 and
bf16 sites) and its optimised plan, and MiniGPT's first kernels
(tests/golden/explain/*.txt, extracted by tests/golden/make_explain.py from
crates/presk-explain/tests/snapshots/documents__*.snap).  Each kernel is
built with the lowering's own functions -- fused groups as the fusion plan
forms them, contractions in the plan's layouts (row form, 2x4 and 4x4 tiles
of 4 lanes), buffers in their sites' types -- and must print character for
character as the reference printed it."""
import os
import re

import pytest

from presk_amd import lower as L

HERE = os.path.dirname(os.path.abspath(__file__))
A, O = L.ax, L.Operand
I0, I1, I2, I3, I4 = ("in", 0), ("in", 1), ("in", 2), ("in", 3), ("in", 4)
S0, S1, S2 = ("step", 0), ("step", 1), ("step", 2)


def fixture(doc):
    """[(header, kernel text)] of a document, in order."""
    out, head, cur = [], None, None
    for line in open(os.path.join(HERE, "golden", "explain", f"{doc}.txt")).read().split("\n"):
        if re.match(r"^// k\d+:", line):
            head, cur = line, []
        elif cur is not None:
            cur.append(line)
            if line == "}":
                out.append((head, "\n".join(cur) + "\n"))
                cur = None
    return out


def tiled(mi, nj, lanes):
    return {"form": "tiled", "tile": (mi, nj), "lanes": lanes}


def sq_diff(a, b, dt):
    """(a - b)^2 as the fusion plan groups it: sub then pow 2"""
    return L.fused([("sub", [I0, I1]), ("pow2", [S0])], [a, b], L.result_axes(a.axes, b.axes), dt).text


def rms_std(r, e, dt):
    """sqrt(ms + eps)"""
    return L.fused([("add", [I0, I1]), ("sqrt", [S0])], [r, e], r.axes, dt).text


def layernorm():
    X, R, E, G = O(A(("batch", 3), ("model", 8))), O(A(("batch", 3))), O(A()), O(A(8))
    return [L.reduce_axis("mean", "model", [X], "f32").text, sq_diff(X, R, "f32"), rms_std(R, E, "f32"),
            L.fused([("sub", [I0, I1]), ("div", [S0, I2]), ("mul", [S1, I3]), ("add", [S2, I4])], [X, R, R, G, G],
                    X.axes, "f32").text]


def linear_add(batch, n_in, n_out, bias_ty, layout):
    x, w, b = O(A(("batch", batch), n_in)), O(A(n_in, n_out)), O(A(n_out), bias_ty)
    d = L.dot([x, w], "f32")
    return L.dot([x, w, b], "f32", layout=layout, epilogue=(True, d.out_axes)).text


def mlp():
    return [linear_add(2, 4, 16, "bf16", tiled(2, 4, 4)), L.unary("gelu", [O(A(("batch", 2), 16))], "f32").text,
            linear_add(2, 16, 4, "bf16", tiled(2, 4, 4)),
            sq_diff(O(A(("batch", 2), 4)), O(A(("batch", 2), ("model", 4))), "f32"),
            L.reduce_all("mean", [O(A(("batch", 2), ("model", 4)), "f32")], "f64").text]


def rmsnorm_block(dt, gamma_ty, dot_text, add_text):
    X, R, E = O(A(("batch", 4), ("model", 4))), O(A(("batch", 4))), O(A())
    return [L.unary("pow2", [X], dt).text, L.reduce_axis("mean", "model", [X], dt).text, rms_std(R, E, dt),
            L.fused([("div", [I0, I1]), ("mul", [S0, I2])], [X, R, O(A(4), gamma_ty)], X.axes, dt).text,
            L.unary("gelu", [X], dt).text] + dot_text + [
            L.elementwise_binary("add", [X, O(A(("batch", 4), 4))], dt).text] + add_text


def tutorial():
    X = O(A(("batch", 4), ("model", 4)))
    return rmsnorm_block("f32", "bf16", [linear_add(4, 4, 4, "bf16", tiled(4, 4, 4))], []) + [
        sq_diff(X, X, "f32"), L.reduce_all("mean", [O(X.axes, "f32")], "f64").text]


def tutorial_typed():
    X = O(A(("batch", 4), ("model", 4)))
    x, w = O(A(("batch", 4), 4), "f32"), O(A(4, 4), "bf16")
    dot = L.dot([O(A(("batch", 4), 4)), w], "f32", layout=tiled(4, 4, 4)).text
    add = L.elementwise_binary("add", [x, O(A(4))], "f64").text
    body = rmsnorm_block("f64", "real", [dot, add], [])
    last = L.fused([("div", [I0, I1]), ("mul", [S0, I2])], [X, O(A(("batch", 4))), O(A(4), "f32")], X.axes, "f64").text
    return body + [last, sq_diff(X, X, "f64"), L.reduce_all("mean", [X], "f64").text]


def tutorial_opt():
    X = O(A(("batch", 4), ("model", 4)))
    dot = L.dot([O(A(("batch", 4), 4)), O(A(4, 4))], "f32", layout={"form": "row", "lanes": 1}).text
    add = L.elementwise_binary("add", [O(A(("batch", 4), 4)), O(A(4))], "f32").text
    return rmsnorm_block("f32", "real", [dot, add], []) + [sq_diff(X, X, "f32"), L.reduce_all("mean", [X], "f32").text]


def minigpt():
    ids = O(A(("batch", 2), ("seq", 8)), "idx")
    return [L.causal_mask("seq", 8, "f32").text, L.embed([O(A(64, 16)), ids], "f32").text, L.positions("seq", 8, "f32").text,
            L.embed([O(A(8, 16)), O(A(("seq", 8)), "idx")], "f32").text,
            L.elementwise_binary("add", [O(A(("batch", 2), ("seq", 8), 16)), O(A(("seq", 8), 16))], "f32").text,
            L.reduce_axis("mean", "model", [O(A(("batch", 2), ("seq", 8), ("model", 16)))], "f32").text]


DOCS = {"layernorm": layernorm, "mlp": mlp, "tutorial": tutorial, "tutorial-typed": tutorial_typed,
        "tutorial-opt": tutorial_opt, "minigpt": minigpt}


@pytest.mark.parametrize("doc", list(DOCS))
def test_kernel_texts_match_the_reference(doc):
    want = fixture(doc)
    got = DOCS[doc]()
    assert len(got) == len(want), (len(got), len(want))
    for (head, w), g in zip(want, got):
        assert g == w, f"{head}\nwant:\n{w}\ngot:\n{g}"
