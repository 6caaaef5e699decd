"""A zoo of the nests the configurations launch, at small shapes, with seeded
inputs: the cases every parity test runs through the oracle and the device."""
from __future__ import annotations

import numpy as np

from presk_amd import lower as L
from tests import fmt

A = L.ax
O = L.Operand


def _gpt_like(dt, B=2, T=8, D=16, H=2, V=11):
    hd = D // H
    x = O(A(("batch", B), ("seq", T), ("model", D)))
    w = O(A(D, D))
    w4 = O(A(D, 4 * D))
    h4 = O(A(("batch", B), ("seq", T), 4 * D))
    b = O(A(D))
    q = O(A(("batch", B), ("heads", H), ("seq", T), ("hd", hd)))
    k = O(A(("batch", B), ("heads", H), ("seq2", T), ("hd", hd)))
    s = O(A(("batch", B), ("heads", H), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    ids = O(A(("batch", B), ("seq", T)), "idx")
    tok = O(A(("vocab", V), ("model", D)))
    logits = O(A(("batch", B), ("seq", T), ("vocab", V)))
    rows = O(A(("batch", B), ("seq", T)))
    d = L.dot([x, w], dt)
    cases = {
        "dot": d,
        "dot+add": L.dot([x, w, b], dt, epilogue=(True, d.out_axes)),
        "dot_vjp_l": L.dot_vjp_l([O(A(("batch", B), ("seq", T), 4 * D)), O(A(D, 4 * D))], dt),
        "dot_vjp_r": L.dot_vjp_r([x, h4], dt),
        "ein_scores": L.ein([q, k], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]], ["batch", "heads", "seq", "seq2"], dt),
        "ein_values": L.ein([s, O(A(("batch", B), ("heads", H), ("seq2", T), ("hd", hd)))],
                            [["batch", "heads", "seq", "seq2"], ["batch", "heads", "seq2", "hd"]], ["batch", "heads", "seq", "hd"], dt),
        "softmax": L.softmax("seq2", [s], dt),
        "softmax2": L.softmax_two_pass("seq2", [s], dt),
        "masked_softmax": L.masked_softmax("seq2", [s, mask], dt),
        "masked_softmax2": L.masked_softmax("seq2", [s, mask], dt, two_passes=True),
        "mean": L.reduce_axis("mean", "model", [x], dt),
        "sum": L.reduce_axis("sum", "model", [x], dt),
        "mean_all": L.reduce_all("mean_all", [rows], dt),
        "sum_squares": L.sum_squares([w4], dt),
        "gelu": L.unary("gelu", [h4], dt),
        "gelu_deriv": L.unary("gelu_deriv", [h4], dt),
        "tanh": L.unary("tanh", [x], dt),
        "sin": L.unary("sin", [x], dt),
        "cos": L.unary("cos", [x], dt),
        "sub": L.elementwise_binary("sub", [x, O(A(("batch", B), ("seq", T)))], dt),
        "max": L.elementwise_binary("max", [x, b], dt),
        "layernorm_tail": L.fused([("sub", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("in", 3)]), ("sqrt", [("step", 1)]),
                                   ("div", [("step", 0), ("step", 2)]), ("mul", [("step", 3), ("in", 4)]), ("add", [("step", 4), ("in", 5)])],
                                  [x, O(A(("batch", B), ("seq", T))), O(A(("batch", B), ("seq", T))), O([]), b, b], x.axes, dt),
        "embed": L.embed([tok, ids], dt),
        "embed_vjp": L.embed_vjp([tok, ids, x], dt),
        "cross_entropy": L.cross_entropy([logits, ids], dt),
        "cross_entropy_vjp": L.cross_entropy_vjp([logits, ids, rows], dt),
        "sum_to": L.sum_to([x, b], dt),
        "sum_to_rows": L.sum_to([x, rows], dt),
        "mean_vjp": L.mean_vjp("model", [rows, x], dt),
        "split_heads": L.split_heads(H, hd, [x], dt),
        "merge_heads": L.merge_heads(H, hd, [q], dt),
        "causal_mask": L.causal_mask("seq", T, dt),
        "positions": L.positions("seq", T, dt),
    }
    return cases


def cases(dtypes=("f32", "bf16", "f16", "e8m15")):
    """[(id, Lowered)] over the zoo and the storage types."""
    out = []
    for dt in dtypes:
        for name, low in _gpt_like(dt).items():
            if dt != "f32" and name in ("causal_mask", "positions"):
                continue
            out.append((f"{name}-{dt}", low))
    # row-wise dot (J % 8 != 0 in f32) and the chunked order
    x = O(A(("batch", 5), 7))
    out.append(("dot_rowwise-f32", L.dot([x, O(A(7, 3))], "f32")))
    out.append(("dot+add_rowwise-f32", L.dot([x, O(A(7, 3)), O(A(3))], "f32", epilogue=(True, A(("batch", 5), 3)))))
    out.append(("dot_chunked4-f32", L.dot([O(A(("batch", 5), 10)), O(A(10, 8))], "f32", order=("chunked", 4))))
    # the declared orders a realization applies to contractions
    # (lower.rs:250-303, 384-475): interleaved on `dot`, chunked on its
    # derivatives and on `ein`
    for dt in ("f32", "bf16", "f16"):
        out.append((f"dot_interleaved4-{dt}", L.dot([O(A(("batch", 5), 12)), O(A(12, 8))], dt, order=("interleaved", 4))))
        out.append((f"dot_interleaved5_ragged-{dt}", L.dot([O(A(("batch", 5), 12)), O(A(12, 8))], dt, order=("interleaved", 5))))
        out.append((f"dot_vjp_l_chunked5-{dt}", L.dot_vjp_l([O(A(("batch", 4), 12)), O(A(7, 12))], dt, order=("chunked", 5))))
        out.append((f"dot_vjp_r_chunked8-{dt}", L.dot_vjp_r([O(A(("batch", 20), 6)), O(A(("batch", 20), 7))], dt, order=("chunked", 8))))
        q = O(A(("heads", 2), ("seq", 5), ("hd", 9)))
        k = O(A(("heads", 2), ("seq2", 5), ("hd", 9)))
        out.append((f"ein_chunked4-{dt}", L.ein([q, k], [["heads", "seq", "hd"], ["heads", "seq2", "hd"]], ["heads", "seq", "seq2"], dt,
                                               order=("chunked", 4))))
    out += _gather_cases()
    return out


def _gather_cases():
    """The dispatch table's remaining nests (lower.rs:1155, 1490-1590,
    1728-1752) and the unary/binary forms of min, max, clamp and their
    derivatives (lower.rs:180-226; rules.rs:115-125: heaviside of a
    difference), in every storage type."""
    out = []
    x = O(A(("batch", 3), ("seq", 5), ("vocab", 7)))
    xi = O(A(("batch", 3), ("seq", 9)), "idx")
    r = O(A(("batch", 3), ("seq", 5)))
    for dt in ("f32", "bf16", "f16", "e8m15"):
        out.append((f"argmax-{dt}", L.argmax([x], dt)))
        out.append((f"index_last-{dt}", L.index_const("seq", -1, [x], dt)))
        out.append((f"index_mid-{dt}", L.index_const("vocab", 3, [x], dt)))
        out.append((f"scatter_index-{dt}", L.scatter_index("seq", -1, [x, O(A(("batch", 3), ("vocab", 7)))], dt)))
        out.append((f"slice-{dt}", L.slice_("vocab", 2, 6, [x], dt)))
        out.append((f"slice_vjp-{dt}", L.slice_vjp("vocab", 2, 6, [x, O(A(("batch", 3), ("seq", 5), ("vocab", 4)))], dt)))
        out.append((f"one_hot-{dt}", L.one_hot(A(("batch", 3), ("seq", 5), ("vocab", 7)), dt)))
        out.append((f"zeros-{dt}", L.fill("zeros", A(("batch", 3), 6), 0.0, dt)))
        out.append((f"ones-{dt}", L.fill("ones", A(("batch", 3), 6), 1.0, dt)))
        for op in ("relu", "heaviside", "sign", "abs"):
            out.append((f"{op}-{dt}", L.unary(op, [x], dt)))
        out.append((f"min-{dt}", L.elementwise_binary("min", [x, r], dt)))
        # clamp(x, lo, hi) = min(max(x, lo), hi) (crates/presk-core/src/lower/expr.rs:540-545)
        out.append((f"clamp-{dt}", L.fused([("max", [("in", 0), ("in", 1)]), ("min", [("step", 0), ("in", 2)])],
                                           [x, O([]), O([])], x.axes, dt)))
        # max's adjoints: heaviside(a - b) * ct and (1 - heaviside(a - b)) * ct
        out.append((f"max_vjp_a-{dt}", L.fused([("sub", [("in", 0), ("in", 1)]), ("heaviside", [("step", 0)]),
                                                ("mul", [("in", 2), ("step", 1)])], [x, x, x], x.axes, dt)))
        out.append((f"max_vjp_b-{dt}", L.fused([("sub", [("in", 0), ("in", 1)]), ("heaviside", [("step", 0)]),
                                                ("sub", [("in", 3), ("step", 1)]), ("mul", [("in", 2), ("step", 2)])],
                                               [x, r, x, O([])], x.axes, dt)))
        # the pack of an NT contraction's operand 1 (lower.rs:1155-1182):
        # dot_vjp_l's matrix and the scores' keys
        c = L.contraction_of("dot_vjp_l", [O(A(("batch", 3), ("seq", 5), 12)), O(A(10, 12))])
        out.append((f"pack_vjp_l-{dt}", L.pack_panel(c, dt, O(A(10, 12)))))
        q = O(A(("batch", 2), ("heads", 3), ("seq", 5), ("hd", 8)))
        k = O(A(("batch", 2), ("heads", 3), ("seq2", 6), ("hd", 8)))
        c = L.contraction_of("ein", [q, k], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]],
                             ["batch", "heads", "seq", "seq2"])
        out.append((f"pack_scores-{dt}", L.pack_panel(c, dt, k)))
    out.append(("slice_idx", L.slice_("seq", 1, 9, [xi], "f32")))
    out.append(("index_idx", L.index_const("seq", 0, [xi], "f32")))
    return out


def inputs(low: L.Lowered, seed: int = 0, scale: float = 1.0):
    """Seeded inputs for a kernel: storage arrays (host) in input order."""
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(seed)
    arrs = []
    for b in k.inputs:
        if b.ty == "i64":
            hi = 2
            if "vocab" in (b.names or []):
                hi = 2
            # an index input: bounded by the axis it indexes in the kernel's use
            hi = _index_bound(low, k, len(arrs))
            arrs.append(rng.integers(0, hi, size=b.numel, dtype=np.int64))
        else:
            v = (rng.standard_normal(b.dims) * scale).astype(np.float32)
            if low.name in ("argmax", "fused 2 steps", "fused 3 steps", "fused 4 steps", "min"):
                # a coarse grid, so that ties (max/min's second operand, the
                # last of equal maxima) and zeros (heaviside's boundary) occur,
                # and a NaN in a first and in a later position
                v = np.round(v * 2).astype(np.float32) / 2
                if low.name == "argmax" and v.size > 8:
                    v.ravel()[0] = np.nan
                    v.ravel()[9] = np.nan
            arrs.append(fmt.encode(v, b.ty))
    return arrs


def _index_bound(low, k, i):
    name = low.name
    if name in ("embed", "embed_vjp"):
        return k.inputs[0].dims[0]
    if name.startswith("cross_entropy"):
        return k.inputs[0].dims[-1]
    if name.startswith("softmax"):
        return 2
    if name == "one_hot":
        # one index past the last position: a row with no hit
        return k.output.dims[-1] + 1
    if name.startswith(("slice", "index")):
        return 1000
    return 2
