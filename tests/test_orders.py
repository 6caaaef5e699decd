"""The reassociating orders a realization declares for its contractions
(`ReductionOrder::Interleaved` and `Chunked`, crates/presk-rt/src/lib.rs:249-
275; nests lower.rs:384-475; which primitive takes which, lower.rs:250-303):
the nests' values in the oracle against brute force sums written from the
orders' definitions, and the rules the reference's own test states
(crates/presk-kernel/tests/formats.rs:359-404): chunks of every size from 1
past the term count, a chunk at least as long as the sum giving the
sequential bits, `ein` and `dot` summing in the same chunks, `dot_vjp_l`
taking the order and `dot_vjp_r` over two summed axes refusing it."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import gpt, hip, llama
from presk_amd import lower as L
from presk_amd.realize import Realization

A, O = L.ax, L.Operand
I, KK, J = 3, 20, 4


def _xw(seed=9):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((I, KK)).astype(np.float32), rng.standard_normal((KK, J)).astype(np.float32)


def _run(low, *ins):
    out, _ = cexec.run(low.text, low.dtype, [np.ascontiguousarray(a).ravel() for a in ins], lanes=low.lanes)
    return out.reshape(I, J)


def _f32_sum(terms):
    s = np.float32(0)
    for t in terms:
        s = np.float32(s + t)
    return s


@pytest.mark.parametrize("c", [1, 3, 8, 20, 32])
def test_chunked_dot_is_its_definition(c):
    x, w = _xw()
    got = _run(L.dot([O(A(("i", I), KK)), O(A(KK, J))], "f32", order=("chunked", c)), x, w)
    for r in range(I):
        for col in range(J):
            terms = [np.float32(x[r, t] * w[t, col]) for t in range(KK)]
            want = _f32_sum([_f32_sum(terms[a:a + c]) for a in range(0, KK, c)])
            assert got[r, col].tobytes() == want.tobytes()
    if c >= KK:
        seq = _run(L.dot([O(A(("i", I), KK)), O(A(KK, J))], "f32"), x, w)
        assert got.tobytes() == seq.tobytes()


@pytest.mark.parametrize("n", [2, 4, 5, 1, 3])
def test_interleaved_dot_is_its_definition(n):
    """n partials, the t-th summing terms t, t+n, ... in order, added left to
    right; an n that does not divide the terms, or 1, is the sequential sum."""
    x, w = _xw(4)
    got = _run(L.dot([O(A(("i", I), KK)), O(A(KK, J))], "f32", order=("interleaved", n)), x, w)
    seq = _run(L.dot([O(A(("i", I), KK)), O(A(KK, J))], "f32"), x, w)
    for r in range(I):
        for col in range(J):
            terms = [np.float32(x[r, t] * w[t, col]) for t in range(KK)]
            if n >= 2 and KK % n == 0:
                parts = [_f32_sum(terms[t::n]) for t in range(n)]
                want = parts[0]
                for p in parts[1:]:
                    want = np.float32(want + p)
            else:
                want = _f32_sum(terms)
            assert got[r, col].tobytes() == want.tobytes()
    if n < 2 or KK % n:
        assert got.tobytes() == seq.tobytes()


def test_which_primitive_takes_which_order():
    x, w = _xw()
    ch = ("chunked", 4)
    e = L.ein([O(A(("i", I), ("k", KK))), O(A(("k", KK), ("j", J)))], [["i", "k"], ["k", "j"]], ["i", "j"], "f32", order=ch)
    d = L.dot([O(A(("i", I), KK)), O(A(KK, J))], "f32", order=ch)
    assert _run(e, x, w).tobytes() == _run(d, x, w).tobytes()
    assert L.dot_vjp_l([O(A(("i", I), J)), O(A(KK, J))], "f32", order=ch).text
    with pytest.raises(ValueError) as err:
        L.dot_vjp_r([O(A(("b", 2), ("t", 3), I)), O(A(("b", 2), ("t", 3), J))], "f32", order=ch)
    assert "chunked(4)" in str(err.value) and "over 2 axes" in str(err.value)
    # interleaved is `dot`'s alone: its derivatives and `ein` keep the exact forms
    il = ("interleaved", 4)
    for low in (L.dot_vjp_l([O(A(("i", I), KK)), O(A(J, KK))], "f32", order=il),
                L.ein([O(A(("i", I), ("k", KK))), O(A(("k", KK), ("j", J)))], [["i", "k"], ["k", "j"]], ["i", "j"], "f32", order=il)):
        assert " = ((" not in low.text     # no partials' index assignments


def test_realization_order_reaches_every_contraction():
    """The GPT forward under interleaved(4): every `dot` an interleaved nest
    (no contraction nest, so no epilogue: the bias `add` its own launch);
    the Llama forward under chunked(8): its `ein`s and `dot`s chunked."""
    r = Realization.of_json({"default": "f32", "order": {"kind": "interleaved", "partials": 4}})
    p, _, _ = gpt.build(gpt.TINY, "f32", train=False, realize=r)
    dots = [ln.low for ln in p.launches if ln.low.name == "dot"]
    assert dots and all("i4 = ((i3 * 4) + 1)" in d.text or "((" in d.text.split("{", 1)[1] for d in dots)
    assert all("+add" not in ln.low.name for ln in p.launches)
    r = Realization.of_json({"default": "f32", "order": {"kind": "chunked", "size": 8}})
    p, _, _ = gpt.build(gpt.TINY, "f32", train=False, mode=hip.EXACT, realize=r)
    conts = [ln.low for ln in p.launches if ln.low.name == "dot" or ln.low.name.startswith("ein[")]
    assert conts and all("s1 = 0" in c.text and " * 8)" in c.text for c in conts)
    # the Llama's RoPE angles are an `ein` with no summed axis, which a
    # chunked order refuses, as the reference's lowering does (lower.rs:611-615)
    with pytest.raises(ValueError, match="0 summed axes"):
        llama.build(llama.TINY, "f32", mode=hip.EXACT, realize=r)
    with pytest.raises(ValueError, match="E7001"):
        Realization.of_json({"default": "f32", "order": {"kind": "spiral"}})


def _lanes_tree_brute(row, vec):
    """FAST's `lanes64xV-tree` from its definition, one row: lane l's
    elements (blocks l, l + 64, ... of `vec` elements) summed in index order
    from +0, then the 64 lane sums added by recursive halving of the lane
    range [0, 64)."""
    f = np.float32
    lane = [f(0.0)] * 64
    for e, x in enumerate(row):
        l = (e // vec) % 64
        lane[l] = f(lane[l] + f(x))

    def tree(lo, hi):
        if hi - lo == 1:
            return lane[lo]
        mid = (lo + hi) // 2
        return f(tree(lo, mid) + tree(mid, hi))
    return tree(0, 64)


@pytest.mark.parametrize("vec,n", [(4, 384), (8, 768), (8, 4096), (1, 65), (4, 8), (8, 2048), (1, 200)])
def test_lanes_tree_order_restatement(vec, n):
    """oracle/lanes.py's vectorized butterfly = the order written from its
    definition (a recursive tree over the lane sums), bit for bit, on rows
    whose terms span 2^20 in magnitude (so that orders differ); and both
    within n u sum|x| of the exact sum."""
    import math
    from oracle.lanes import lanes_tree_sum
    rng = np.random.default_rng(n + vec)
    x = (rng.standard_normal((6, n)) * np.exp2(rng.integers(-10, 10, (6, n)))).astype(np.float32)
    got = lanes_tree_sum(x, vec)
    for r in range(6):
        assert got[r] == _lanes_tree_brute(x[r], vec), (r, got[r], _lanes_tree_brute(x[r], vec))
        exact = math.fsum(float(v) for v in x[r])
        assert abs(float(got[r]) - exact) <= (n + 64) * 2.0 ** -24 * float(np.abs(x[r].astype(np.float64)).sum())
    # an order, not the sequential one: some row differs from the in-order sum
    seq = np.zeros(6, np.float32)
    for e in range(n):
        seq = seq + x[:, e]
    assert n <= 8 or np.any(seq != got)
