"""Integer weights on the host and in the oracle.

- The quantiser (presk_amd/quant.py) against the reference's own known
  answers and rules (crates/presk-rt/tests/quant.rs): absmax's error rule and
  full range, pow2's exact products and minimal scales, int4 packing of
  [7, -7, 0, 3, -1, 5, -4], a zero channel, per-layer scales of a stacked
  parameter, refused axes and bit widths.
- `of_quant` (crates/presk-kernel/src/ir.rs:52-79) on a stored axis kept and
  split by a view.
- The oracle's integer loads (f32(q) * s, the channel from the flat index)
  against brute force on tiny kernels, and the executor's reader printing
  the `int8/o` and `int4/o..e` types back.
"""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from presk_amd import quant as Q

A, O = L.ax, L.Operand


def weights(dims):
    """quant.rs:14-19's deterministic tensor: octaves of magnitude, mixed signs."""
    n = int(np.prod(dims))
    i = np.arange(n)
    return ((i * 7919 % 101) - 50.0) / 37.0 * (1.0 + (i % 5))


@pytest.mark.parametrize("bits", [8, 4])
def test_absmax_meets_its_error_rule(bits):
    w = weights((16, 6))
    qt = Q.quantize(w, (16, 6), Q.Quant(bits, -2))
    assert qt.scales.size == 6
    d = qt.dequantize().astype(np.float64)
    s = qt.scales[qt.channels()].astype(np.float64)
    assert np.all(np.abs(w - d) <= s / 2 + np.abs(d) * 2.0 ** -24)
    q = qt.ints()
    assert np.all(np.abs(q) <= qt.quant.qmax)
    assert np.all(np.abs(q.reshape(16, 6)).max(axis=0) == qt.quant.qmax)


def test_pow2_scales_are_exact():
    w = weights((12, 5))
    qt = Q.quantize(w, (12, 5), Q.Quant(8, "model", Q.POW2), names=["model", "vocab"])
    d = qt.dequantize().astype(np.float64)
    s = qt.scales[qt.channels()].astype(np.float64)
    assert np.all(np.log2(s) == np.round(np.log2(s)))
    assert np.array_equal(d, qt.ints().astype(np.float64) * s)
    assert np.all(np.abs(w - d) <= s / 2)
    m = np.abs(w.reshape(12, 5)).max(axis=0)
    assert np.all(m / qt.scales <= 127) and np.all(m / (qt.scales / 2.0) > 127)


def test_int4_packs_two_to_a_byte():
    v = np.array([7.0, -7.0, 0.0, 3.0, -1.0, 5.0, -4.0])
    qt = Q.quantize(v, (7, 1), Q.Quant(4, 0))
    assert qt.data.size == 4
    assert qt.scales.tolist() == [1.0]
    assert qt.ints().tolist() == [7, -7, 0, 3, -1, 5, -4]
    assert qt.dequantize().tolist() == v.astype(np.float32).tolist()


def test_a_zero_channel_stays_zero():
    qt = Q.quantize([0.0, 1.0, 0.0, -2.0, 0.0, 0.5], (3, 2), Q.Quant(8, 0))
    assert qt.scales[0] == 0.0
    d = qt.dequantize()
    assert d[[0, 2, 4]].tolist() == [0.0, 0.0, 0.0] and np.all(np.isfinite(d))


def test_stacked_parameters_get_scales_per_layer():
    w = weights((2, 4, 3))
    w[12:] = w[:12] * 100.0
    qt = Q.quantize(w, (2, 4, 3), Q.Quant(8, -2))
    assert qt.over == 1 and qt.scales.size == 6
    assert np.all(np.abs(qt.scales[3:] / qt.scales[:3] - 100.0) < 1e-3)


def test_a_bad_axis_is_refused():
    w = weights((2, 2))
    for q, names in [(Q.Quant(8, "a"), ["a", "a"]), (Q.Quant(8, "b"), ["a", "a"]), (Q.Quant(8, 2), None), (Q.Quant(6, 0), None)]:
        with pytest.raises(ValueError):
            Q.quantize(w, (2, 2), q, names=names)


def test_of_quant_kept_and_split_axes():
    qt = Q.quantize(weights((8, 6)), (8, 6), Q.Quant(8, 0))     # scales constant along axis 0 (k 8, inner 6)
    assert Q.of_quant(qt, (8, 6)) == (8, 0, 1)
    assert Q.of_quant(qt, (2, 4, 6)) == (8, 0, 2)                # the view splits the stored axis
    assert Q.of_quant(qt, (2, 4, 2, 3)) == (8, 0, 2)
    assert Q.of_quant(qt, (48,)) is None                        # merged with another axis


def _dot_case(bits, span, dt, lanes=1):
    """x[5, K] . w[K, 3] with w quantised along K, K = 8 as one axis or as
    (2, 4) through a split view (an `ein` over two summed axes)."""
    rng = np.random.default_rng(bits + span)
    w = rng.standard_normal((8, 3))
    qt = Q.quantize(w, (8, 3), Q.Quant(bits, 0))
    x = rng.standard_normal((5, 8)).astype(np.float32)
    if span == 1:
        low = L.dot([O(A(("batch", 5), 8)), O(A(8, 3))], dt)
        kind = Q.of_quant(qt, (8, 3))
    else:
        low = L.ein([O(A(("batch", 5), ("a", 2), ("b", 4))), O(A(("a", 2), ("b", 4), ("out", 3)))],
                    [["batch", "a", "b"], ["a", "b", "out"]], ["batch", "out"], dt)
        kind = Q.of_quant(qt, (2, 4, 3))
    assert kind == (bits, 0, span)
    return Q.mark(low.text, 1, kind), x, qt


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("span", [1, 2])
def test_oracle_loads_f32_q_times_scale(bits, span):
    text, x, qt = _dot_case(bits, span, "f32")
    out, _ = cexec.run(text, "f32", [x.ravel(), (qt.data, qt.scales)])
    # brute force: the dequantised weights, the sum over K in index order in f32
    wv = qt.dequantize().reshape(8, 3)
    want = np.zeros((5, 3), np.float32)
    for i in range(5):
        for j in range(3):
            acc = np.float32(0)
            for kk in range(8):
                acc = np.float32(acc + np.float32(x[i, kk] * wv[kk, j]))
            want[i, j] = acc
    assert np.array_equal(out.reshape(5, 3), want)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("span", [1, 2])
def test_reader_prints_integer_types_back(bits, span):
    text, _, _ = _dot_case(bits, span, "f32")
    assert (f"int{bits}/0" + ("..2" if span == 2 else "") + "[") in text
    for mode in (hip.EXACT, hip.FAST):
        c = hip.Compiled(text, "f32", 1, mode)
        assert c.read_back() == text
        # EXACT: the generic printer's loads; FAST: the f32 MFMA kernel on them
        assert c.kind == ("generic" if mode == hip.EXACT else "gemm"), (mode, c.kind)
        # the scales' slot after the output counts in the table's length: a
        # table of the inputs and the output alone is refused on the host
        assert c.n_inputs == 2 and c.n_quant == 1
        with pytest.raises(ValueError, match="1 integer, with scales"):
            c.run([0x1000, 0x2000, 0x3000])


def test_integer_output_is_malformed():
    text = ("kernel neg (%0 : f32[2]) -> %1 : int8/0[2] {\n  for i0 in 0..2 {\n    %1[i0] = (-%0[i0])\n  }\n}\n")
    with pytest.raises(hip.HipError) as e:
        hip.Compiled(text, "f32")
    assert e.value.code == "E10001"


# ---- the realization's `quant` map on whole programs -------------------------

from presk_amd import gpt, llama                      # noqa: E402
from presk_amd.realize import Realization           # noqa: E402
from tests import cpu_program                       # noqa: E402

QUANT_LLAMA = {"blocks.attn.wq": {"bits": 8, "over": -2}, "blocks.attn.wo": {"bits": 8, "over": -2},
               "blocks.ff.down.w": {"bits": 4, "over": -2}, "head": {"bits": 8, "over": -2, "scheme": "pow2"}}


def _dequantized_host(p, host):
    """The host's weights replaced by the values the realization denotes,
    f32(q) * s (quant.rs:177-182), each quantised as the program stores it."""
    env = cpu_program.storage_of(host, p)
    out = dict(host)
    for name, (q, over, axes) in p.quant.items():
        qt = Q.QTensor(tuple(a.len for a in axes), over, q, env[name + "#scales"], env[name])
        out[name] = qt.dequantize().reshape([a.len for a in axes])
    return out


def test_quantised_llama_equals_dequantised_weights():
    """In f32 storage a load of an integer weight is f32(q) * s, exactly the
    f32 value of the dequantised weight: the quantised program's every
    buffer equals the plain program's fed those values -- which pins the
    marking of each reader (a split view's span included: the output
    projection reads `wo` as int8/0..3), the scales' slots and the channels."""
    s = llama.TINY
    r = Realization.of_json({"default": "f32", "order": {"kind": "sequential"}, "quant": QUANT_LLAMA})
    pq, _, names = llama.build(s, "f32", mode=hip.EXACT, realize=r)
    texts = [ln.low.text.split("\n", 1)[0] for ln in pq.launches]
    assert any("int8/0..3[" in t for t in texts) and any("int4/0[" in t for t in texts)
    assert sum(len(ln.scales) for ln in pq.launches) == 3 * s.L + 1     # wq, wo, down a layer; the head
    host = llama.host_inputs(s)
    envq = cpu_program.run(pq, host)
    p0, _, _ = llama.build(s, "f32", mode=hip.EXACT)
    env0 = cpu_program.run(p0, _dequantized_host(pq, host))
    bad = [ln.out for ln in p0.launches if env0[ln.out].tobytes() != envq[ln.out].tobytes()]
    assert not bad, bad[:5]


def test_realization_paths_are_the_trees():
    """`params` and `quant` are keyed by the parameter's dotted path; a path
    the program does not have is refused (E7001, presk-rt lib.rs:697-701), a
    stacked path names every layer, and a path in both maps is refused."""
    s = gpt.TINY
    r = Realization.of_json({"default": "f32", "order": {"kind": "sequential"},
                             "params": {"blocks.attn.wq.w": "bf16", "lnf.γ": "f16"}})
    p, _, _ = gpt.build(s, "f32", train=False, realize=r)
    assert all(p.input_types[f"b{l}.wq"] == "bf16" for l in range(s.L))
    assert p.input_types["lnf.g"] == "f16" and p.input_types["b0.wk"] == "f32"
    for bad in ({"params": {"b0.wq": "bf16"}}, {"quant": {"blocks.wq": {"bits": 8, "over": -2}}}):
        with pytest.raises(ValueError, match="E7001"):
            gpt.build(s, "f32", train=False, realize=Realization.of_json({"default": "f32", "order": {"kind": "sequential"}, **bad}))
    with pytest.raises(ValueError, match="E7001"):
        Realization.of_json({"default": "f32", "order": {"kind": "sequential"}, "params": {"head": "bf16"},
                             "quant": {"head": {"bits": 8, "over": -2}}})
    with pytest.raises(ValueError, match="E7001"):
        Realization.of_json({"default": "f32", "order": {"kind": "sequential"}, "quant": {"head": {"bits": 6, "over": 0}}})
