"""The oracle's runs of the dispatch table's gathers, scatters, packs and
selects (presk_amd/lower.py's restatements of lower.rs:1155-1182,
1490-1590, 1728-1752 and the min/max/clamp forms of lower.rs:180-226)
against numpy written from each primitive's definition: argmax keeps the
last of equal maxima and passes over a later NaN, while a NaN at element 0
keeps position 0 (the nest's `>=` from element 0), `index` drops its axis and counts a negative index from the end,
`scatter_index`/`slice_vjp` put the cotangent into zeros, `one_hot` is 1 at
the index's position, a pack is the transposed panel, `max`/`min` pick the
second operand on a tie, `clamp` is min(max(x, lo), hi)."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import lower as L
from tests import fmt, zoo

A, O = L.ax, L.Operand
DTS = ("f32", "bf16", "f16", "e8m15")


def run(low, ins):
    out, flag = cexec.run(low.text, low.dtype, ins, lanes=low.lanes)
    assert not flag
    return out


def values(ins, low, i):
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    b = k.inputs[i]
    return fmt.decode(ins[i], low.dtype).astype(np.float64).reshape(b.dims) if b.ty != "i64" else ins[i].reshape(b.dims)


def result(out, low):
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    if k.output.ty == "i64":
        return out.reshape(k.output.dims)
    return fmt.decode(out, low.dtype).astype(np.float64).reshape(k.output.dims)


def argmax_last(x):
    """The last position of the row's maximum, walked from element 0 with
    `>=` (a NaN compares false either way)."""
    out = np.zeros(x.shape[:-1], np.int64)
    for ix in np.ndindex(*x.shape[:-1]):
        row = x[ix]
        m, best = row[0], 0
        for k in range(len(row)):
            if row[k] >= m:
                m, best = row[k], k
        out[ix] = best
    return out


@pytest.mark.parametrize("dt", DTS)
def test_argmax_last_of_ties_skips_nans(dt):
    x = O(A(("batch", 3), ("seq", 5), ("vocab", 7)))
    low = L.argmax([x], dt)
    ins = zoo.inputs(low, seed=1)
    v = values(ins, low, 0)
    got = result(run(low, ins), low)
    # brute force over the reference's rule, then the closed forms it reduces to
    assert np.array_equal(got, argmax_last(v))
    clean = ~np.isnan(v).any(axis=-1)
    rev = v.shape[-1] - 1 - np.argmax(v[..., ::-1], axis=-1)     # numpy's argmax is the first maximum
    assert np.array_equal(got[clean], rev[clean])
    assert np.isnan(v).any() and (v == np.roll(v, 1, axis=-1)).any(), "the sample holds NaNs and ties"


@pytest.mark.parametrize("dt", DTS)
def test_index_scatter_slice_one_hot(dt):
    x = O(A(("batch", 3), ("seq", 5), ("vocab", 7)))
    rng = np.random.default_rng(2)
    xv = fmt.roundtrip(rng.standard_normal((3, 5, 7)).astype(np.float32), dt).astype(np.float64)
    xs = fmt.encode(xv.astype(np.float32), dt)
    low = L.index_const("seq", -1, [x], dt)
    assert np.array_equal(result(run(low, [xs]), low), xv[:, -1, :])
    low = L.index_const("vocab", 3, [x], dt)
    assert np.array_equal(result(run(low, [xs]), low), xv[:, :, 3])
    ct = fmt.roundtrip(rng.standard_normal((3, 7)).astype(np.float32), dt).astype(np.float64)
    low = L.scatter_index("seq", -1, [x, O(A(("batch", 3), ("vocab", 7)))], dt)
    want = np.zeros((3, 5, 7))
    want[:, 4, :] = ct
    assert np.array_equal(result(run(low, [xs, fmt.encode(ct.astype(np.float32), dt)]), low), want)
    low = L.slice_("vocab", 2, 6, [x], dt)
    assert np.array_equal(result(run(low, [xs]), low), xv[:, :, 2:6])
    ct4 = fmt.roundtrip(rng.standard_normal((3, 5, 4)).astype(np.float32), dt).astype(np.float64)
    low = L.slice_vjp("vocab", 2, 6, [x, O(A(("batch", 3), ("seq", 5), ("vocab", 4)))], dt)
    want = np.zeros((3, 5, 7))
    want[:, :, 2:6] = ct4
    assert np.array_equal(result(run(low, [xs, fmt.encode(ct4.astype(np.float32), dt)]), low), want)
    idx = rng.integers(0, 8, size=(3, 5)).astype(np.int64)
    low = L.one_hot(A(("batch", 3), ("seq", 5), ("vocab", 7)), dt)
    assert np.array_equal(result(run(low, [idx]), low), (idx[..., None] == np.arange(7)).astype(np.float64))
    low = L.fill("ones", A(("batch", 3), 6), 1.0, dt)
    assert np.array_equal(result(run(low, []), low), np.ones((3, 6)))


def test_index_tensors_copied_as_indices():
    xi = O(A(("batch", 3), ("seq", 9)), "idx")
    w = np.arange(27, dtype=np.int64).reshape(3, 9) * 7 + 1
    low = L.slice_("seq", 1, 9, [xi], "f32")
    assert low.out_kind == "idx" and "-> %1 : i64[batch: 3, seq: 8]" in low.text
    assert np.array_equal(result(run(low, [w.ravel()]), low), w[:, 1:])
    low = L.index_const("seq", 0, [xi], "f32")
    assert np.array_equal(result(run(low, [w.ravel()]), low), w[:, 0])


@pytest.mark.parametrize("dt", DTS)
def test_min_max_clamp_and_their_adjoints(dt):
    rng = np.random.default_rng(3)
    shape = (3, 5, 7)
    grid = lambda: fmt.roundtrip((np.round(rng.standard_normal(shape) * 2) / 2).astype(np.float32), dt).astype(np.float64)
    a, b, ct = grid(), grid(), grid()
    x = O(A(("batch", 3), ("seq", 5), ("vocab", 7)))
    enc = lambda v: fmt.encode(np.asarray(v, np.float32), dt)
    low = L.elementwise_binary("max", [x, x], dt)
    assert np.array_equal(result(run(low, [enc(a), enc(b)]), low), np.where(a > b, a, b))
    low = L.elementwise_binary("min", [x, x], dt)
    assert np.array_equal(result(run(low, [enc(a), enc(b)]), low), np.where(a < b, a, b))
    assert (a == b).any(), "the sample holds ties"
    lo, hi = np.array([-0.5]), np.array([1.0])
    low = L.fused([("max", [("in", 0), ("in", 1)]), ("min", [("step", 0), ("in", 2)])], [x, O([]), O([])], x.axes, dt)
    assert np.array_equal(result(run(low, [enc(a), enc(lo), enc(hi)]), low), np.clip(a, -0.5, 1.0))
    # rules.rs:115-125: u = heaviside(a - b); a's cotangent ct * u, b's ct * (1 - u)
    u = (a - b > 0).astype(np.float64)
    low = L.fused([("sub", [("in", 0), ("in", 1)]), ("heaviside", [("step", 0)]), ("mul", [("in", 2), ("step", 1)])],
                  [x, x, x], x.axes, dt)
    assert np.array_equal(result(run(low, [enc(a), enc(b), enc(ct)]), low), fmt.roundtrip((ct * u).astype(np.float32), dt))
    for op, f in (("relu", lambda v: np.maximum(v, 0)), ("heaviside", lambda v: (v > 0) * 1.0),
                  ("sign", np.sign), ("abs", np.abs)):
        low = L.unary(op, [x], dt)
        assert np.array_equal(result(run(low, [enc(a)]), low), f(a)), op


def test_pack_panels_are_transposes():
    c = L.contraction_of("dot_vjp_l", [O(A(("batch", 3), ("seq", 5), 12)), O(A(10, 12))])
    low = L.pack_panel(c, "f32", O(A(10, 12)))
    w = np.arange(120, dtype=np.float32).reshape(10, 12)
    assert low.name == "pack" and low.out_axes == A(12, 10)
    assert np.array_equal(result(run(low, [w.ravel()]), low), w.T)
    q = O(A(("batch", 2), ("heads", 3), ("seq", 5), ("hd", 8)))
    k = O(A(("batch", 2), ("heads", 3), ("seq2", 6), ("hd", 8)))
    c = L.contraction_of("ein", [q, k], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]],
                         ["batch", "heads", "seq", "seq2"])
    low = L.pack_panel(c, "bf16", k)
    assert low.out_axes == A(("batch", 2), ("heads", 3), ("hd", 8), ("seq2", 6))
    kv = np.random.default_rng(4).standard_normal((2, 3, 6, 8)).astype(np.float32)
    ks = fmt.encode(kv, "bf16")
    got = result(run(low, [ks]), low)
    assert np.array_equal(got, fmt.roundtrip(kv, "bf16").transpose(0, 1, 3, 2))
    # the packed contraction reads the panel as NN and gives the same sum
    pc = L.packed(c)
    assert pc.w_index == [("o", 0), ("o", 1), "K", "J"] and not pc.nt
