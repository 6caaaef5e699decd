"""The course GPT (examples/corpus/nlp/05_gpt.psk) as programs of the
reference's nests: config 3 (forward and loss) and config 4 (one training
step: the loss's value and its gradient in every parameter, `value_vjp`).

The forward is the program's `GPT.apply` and `loss`: token and position
embeddings, L pre-LayerNorm blocks of causal self-attention (split_heads,
`ein` scores, the 1/sqrt(HD) scale, the masked softmax, `ein` values,
merge_heads) and a GELU MLP, a final LayerNorm, the head `dot`, and
`mean(cross_entropy(...))`.  Dropout is at p = 0 (the configs' reading).

The gradient restates the reference's reverse mode: each primitive's
vector-Jacobian product as crates/presk-core/src/ad/rules.rs:16-217 emits it
(`dot` -> `dot_vjp_l` + `dot_vjp_r`; `ein` -> one `ein` per operand;
broadcast adds -> `sum_to`; `mean` -> `mean_vjp`; `softmax` ->
`y * (ct - broadcast(sum(ct * y)))`; `gelu` -> `gelu_deriv * ct`; `embed` ->
`embed_vjp`; `cross_entropy` -> `cross_entropy_vjp`; split/merge_heads ->
each other), cotangents of a value used twice added.  Elementwise chains are
grouped as the fusion plan groups them (crates/presk-core/src/fusion.rs:
138): a chain of one result type whose interior values have one consumer is
one `fused` nest.  The reference's exact grouping of the gradient entry and
its layout plan can only be read off `presk dump`, which needs the Rust
reference; this restatement is pinned by its mathematics instead (the
gradient against torch autograd, tests/test_gpt_program.py).
"""
from __future__ import annotations

import contextlib
import dataclasses
import math
import re
from dataclasses import dataclass

import numpy as np

from . import lower as L
from . import fusion as FU
from . import quant as Q
from .fusion import Let
from .program import Program

A, O = L.ax, L.Operand


@dataclass
class GptShape:
    V: int = 65
    D: int = 384
    H: int = 6
    L: int = 6
    B: int = 64
    T: int = 256

    @property
    def HD(self):
        return self.D // self.H


TINY = GptShape(V=64, D=16, H=2, L=2, B=2, T=8)
COURSE = GptShape()


class Builder:
    """Buffers by name with their axes and kind; each primitive one launch.

    Each launch is a site, `<function>/<let>` (crates/presk-rt/src/lib.rs:370-373):
    the function is the builder's current one (`func`), the let the result's
    name.  Its storage type is the realization's for the site when one is
    given (`Realization.dtype_at`), else the builder's one type."""

    def __init__(self, prog: Program, dtype: str, realize=None):
        self.p, self.dt, self.realize = prog, dtype, realize
        self.axes: dict = {}
        self.kind: dict = {}
        # a view's buffer (`split`/`merge` read one buffer under other axes,
        # crates/presk-kernel/src/host.rs:1510-1536: no launch)
        self.base: dict = {}
        self.n = 0
        self.fn = "MiniGPT.apply"

    @contextlib.contextmanager
    def func(self, name: str):
        prev, self.fn = self.fn, name
        try:
            yield
        finally:
            self.fn = prev

    def input(self, name, axes, kind="real"):
        self.axes[name], self.kind[name] = list(axes), kind
        return name

    def op(self, name):
        return O(self.axes[name], self.kind[name])

    def _name(self, name):
        if name is None:
            self.n += 1
            name = f"t{self.n}"
        return name

    def _dt(self, name):
        """The site's storage type; the site's let is the result's name
        without its layer (`b3.scores` -> `scores`), so that one entry names a
        let of every layer, as a site of a function does in the reference."""
        if self.realize is None:
            return self.dt
        return self.realize.dtype_at(f"{self.fn}/{re.sub(r'^b[0-9]+[.]', '', name)}")

    def view(self, src, axes, name=None):
        """`src` under other axes of the same element count, no launch."""
        name = self._name(name)
        n0 = 1
        for a in self.axes[src]:
            n0 *= a.len
        n1 = 1
        for a in axes:
            n1 *= a.len
        if n0 != n1:
            raise ValueError(f"view {name}: {n1} elements of {src}'s {n0}")
        self.axes[name], self.kind[name] = list(axes), self.kind[src]
        self.base[name] = self.base.get(src, src)
        return name

    def split(self, src, axis, n1, l1, n2, l2, name=None):
        """`split(axis a, n1: l1, n2: l2, x)` (host.rs:1523-1536)."""
        ax = self.axes[src]
        p = next(i for i, a in enumerate(ax) if a.name == axis)
        if l1 * l2 != ax[p].len:
            raise ValueError(f"split: `{axis}` has length {ax[p].len}")
        return self.view(src, ax[:p] + [L.Axis(n1, l1), L.Axis(n2, l2)] + ax[p + 1:], name)

    def merge(self, src, a, b_, name=None):
        """`merge(axis a, axis b, x)` (host.rs:1510-1522): the joined axis is unnamed."""
        ax = self.axes[src]
        p = next(i for i, x in enumerate(ax) if x.name == a)
        if p + 1 >= len(ax) or ax[p + 1].name != b_:
            raise ValueError(f"merge: `{a}` is not immediately followed by `{b_}`")
        return self.view(src, ax[:p] + [L.Axis(None, ax[p].len * ax[p + 1].len)] + ax[p + 2:], name)

    def _out(self, low, ins, name):
        # an input holding integer weights is marked with its buffer kind,
        # the run of the view's axes its scales are constant along
        # (BufKind::of_quant, crates/presk-kernel/src/ir.rs:52-79), and its
        # scales ride after the output
        scales = []
        for j, i in enumerate(ins):
            base = self.base.get(i, i)
            if base not in self.p.quant:
                continue
            q, over, axes = self.p.quant[base]
            kind = Q.of_quant_dims(q.bits, over, [a.len for a in axes], [a.len for a in self.axes[i]])
            if kind is None:
                raise ValueError(f"E7005: `{low.name}` reads the integer weights `{base}` through a view that merges "
                                 f"their quantised axis")
            low = dataclasses.replace(low, text=Q.mark(low.text, j, kind))
            scales.append(base + "#scales")
        self.p.add(low, [self.base.get(i, i) for i in ins], name, scales)
        self.axes[name], self.kind[name] = list(low.out_axes), low.out_kind
        return name

    def _prim(self, make, ins, name):
        """One primitive: `make(dtype)` lowers it at the site's storage type."""
        name = self._name(name)
        return self._out(make(self._dt(name)), ins, name)

    def params_of(self, leaves: dict, rename: dict, shapes: dict):
        """The realization's `params` types and `quant` weights on the
        program's parameter buffers, by their dotted paths (E7001 for a path
        the program does not have)."""
        types, quants = self.realize.resolve_params(leaves, rename)
        for name in shapes:
            self.p.input_types[name] = types.get(name, "f32")
        for name, (q, over, axes) in quants.items():
            self.p.input_types[name] = f"int{q.bits}"
            self.p.quant[name] = (q, over, axes)

    # --- primitives -----------------------------------------------------------
    def binary(self, op, a, b, name=None):
        return self._prim(lambda dt: L.elementwise_binary(op, [self.op(a), self.op(b)], dt), [a, b], name)

    def unary(self, op, a, name=None):
        return self._prim(lambda dt: L.unary(op, [self.op(a)], dt), [a], name)

    def fused(self, steps, ins, out_like, name=None):
        return self._prim(lambda dt: L.fused(steps, [self.op(i) for i in ins], self.axes[out_like], dt), ins, name)

    def order(self):
        """The realization's reduction order, applied to the contractions as
        `lower_planned` applies it (lower.rs:250-303); None when exact."""
        return L.order_of(self.realize.order) if self.realize is not None else None

    def dot(self, x, w, b=None, name=None):
        o = self.order()
        if b is not None and not L.exact_order(o):
            # no contraction nest under a reassociating order, so no epilogue:
            # the product and the `add` are two launches
            name = self._name(name)
            d = self._prim(lambda dt: L.dot([self.op(x), self.op(w)], dt, order=o), [x, w], name + ".dot")
            return self.binary("add", d, b, name=name)

        def make(dt):
            d = L.dot([self.op(x), self.op(w)], dt, order=o)
            if b is None:
                return d
            return L.dot([self.op(x), self.op(w), self.op(b)], dt, epilogue=(True, d.out_axes))
        return self._prim(make, [x, w] if b is None else [x, w, b], name)

    def dot_vjp_l(self, ct, b, name=None):
        return self._prim(lambda dt: L.dot_vjp_l([self.op(ct), self.op(b)], dt, order=self.order()), [ct, b], name)

    def dot_vjp_r(self, a, ct, name=None):
        return self._prim(lambda dt: L.dot_vjp_r([self.op(a), self.op(ct)], dt, order=self.order()), [a, ct], name)

    def ein(self, a, b, la, lb, out, name=None, like=None):
        """`like`: the value whose type the result has -- an operand's, for the
        `ein` of its cotangent (rules.rs:151-169 gives it `tys[j]`)."""
        r = self._prim(lambda dt: L.ein([self.op(a), self.op(b)], [la, lb], out, dt, order=self.order()), [a, b], name)
        if like is not None:
            self.axes[r] = list(self.axes[like])
        return r

    def mean(self, x, axis, name=None):
        return self._prim(lambda dt: L.reduce_axis("mean", axis, [self.op(x)], dt), [x], name)

    def sum(self, x, axis, name=None):
        return self._prim(lambda dt: L.reduce_axis("sum", axis, [self.op(x)], dt), [x], name)

    def mean_all(self, x, name=None):
        return self._prim(lambda dt: L.reduce_all("mean_all", [self.op(x)], dt), [x], name)

    def mean_vjp(self, ct, like, axis, name=None):
        return self._prim(lambda dt: L.mean_vjp(axis, [self.op(ct), self.op(like)], dt), [ct, like], name)

    def sum_to(self, x, like, name=None):
        return self._prim(lambda dt: L.sum_to([self.op(x), self.op(like)], dt), [x, like], name)

    def broadcast_like(self, x, like, name=None):
        return self._prim(lambda dt: L.broadcast_like([self.op(x), self.op(like)], dt), [x, like], name)

    def masked_softmax(self, x, mask, axis, name=None):
        return self._prim(lambda dt: L.masked_softmax(axis, [self.op(x), self.op(mask)], dt), [x, mask], name)

    def embed(self, table, ids, name=None):
        out = self._prim(lambda dt: L.embed([self.op(table), self.op(ids)], dt), [table, ids], name)
        # the result's last axis is the table's (its type names it)
        last = self.axes[table][-1]
        self.axes[out][-1] = L.Axis(last.name, last.len)
        return out

    def embed_vjp(self, table, ids, ct, name=None):
        return self._prim(lambda dt: L.embed_vjp([self.op(table), self.op(ids), self.op(ct)], dt), [table, ids, ct], name)

    def split_heads(self, x, h, hd, name=None):
        return self._prim(lambda dt: L.split_heads(h, hd, [self.op(x)], dt), [x], name)

    def merge_heads(self, x, h, hd, name=None):
        return self._prim(lambda dt: L.merge_heads(h, hd, [self.op(x)], dt), [x], name)

    def cross_entropy(self, logits, y, name=None):
        return self._prim(lambda dt: L.cross_entropy([self.op(logits), self.op(y)], dt), [logits, y], name)

    def cross_entropy_vjp(self, logits, y, ct, name=None):
        return self._prim(lambda dt: L.cross_entropy_vjp([self.op(logits), self.op(y), self.op(ct)], dt), [logits, y, ct], name)

    def dropout_mask(self, x, slot: int, rate: float, name=None):
        """`DropoutMask(rate, key, x)`: a mask of x's shape and the site's
        type, drawn from key `slot` of the program's key table."""
        name = self._name(name)
        n = 1
        for a in self.axes[x]:
            n *= a.len
        self.p.add_mask(name, slot, rate, self._dt(name), n)
        self.axes[name], self.kind[name] = list(self.axes[x]), "real"
        return name

    def slice(self, x, axis, lo, hi, name=None):
        return self._prim(lambda dt: L.slice_(axis, lo, hi, [self.op(x)], dt), [x], name)

    def slice_vjp(self, tmpl, ct, axis, lo, hi, name=None):
        return self._prim(lambda dt: L.slice_vjp(axis, lo, hi, [self.op(tmpl), self.op(ct)], dt), [tmpl, ct], name)

    def index(self, x, axis, i, name=None):
        return self._prim(lambda dt: L.index_const(axis, i, [self.op(x)], dt), [x], name)

    def scatter_index(self, tmpl, ct, axis, i, name=None):
        return self._prim(lambda dt: L.scatter_index(axis, i, [self.op(tmpl), self.op(ct)], dt), [tmpl, ct], name)

    def argmax(self, x, name=None):
        return self._prim(lambda dt: L.argmax([self.op(x)], dt), [x], name)

    def concat(self, x, y, axis, name=None):
        return self._prim(lambda dt: L.concat(axis, [self.op(x), self.op(y)], dt), [x, y], name)

    def causal_mask(self, T, name):
        return self._prim(lambda dt: L.causal_mask("seq", T, dt), [], name)

    def positions(self, T, name, axis="seq"):
        return self._prim(lambda dt: L.positions(axis, T, dt), [], name)


def param_shapes(s: GptShape) -> dict:
    """name -> axes of every parameter (05_gpt.psk's modules)."""
    ps = {"tok": A(("vocab", s.V), ("model", s.D)), "pos": A(s.T, s.D)}
    for l in range(s.L):
        p = f"b{l}."
        for ln in ("ln1", "ln2"):
            ps[p + ln + ".g"] = A(("model", s.D))
            ps[p + ln + ".b"] = A(("model", s.D))
        for w in ("wq", "wk", "wv", "wo"):
            ps[p + w] = A(s.D, s.D)
            ps[p + w + ".b"] = A(s.D)
        ps[p + "up"] = A(s.D, 4 * s.D)
        ps[p + "up.b"] = A(4 * s.D)
        ps[p + "down"] = A(4 * s.D, s.D)
        ps[p + "down.b"] = A(s.D)
    ps["lnf.g"] = A(("model", s.D))
    ps["lnf.b"] = A(("model", s.D))
    ps["head"] = A(s.D, s.V)
    return ps


def init_params(s: GptShape, seed: int = 2) -> dict:
    """Config 3's weights: N(0, 0.02) for every weight matrix and embedding,
    LayerNorm gains one and biases zero, linear biases N(0, 0.02) (the
    program's zeros would make the bias gradients' checks vacuous)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, axes in param_shapes(s).items():
        shape = [a.len for a in axes]
        if name.endswith(".g"):
            out[name] = np.ones(shape, np.float32)
        elif name.endswith(".b") and (".ln" in name or name.startswith("lnf")):
            out[name] = np.zeros(shape, np.float32)
        else:
            out[name] = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    return out


def _layernorm(b: Builder, x, g, bias, keep: bool, tag: str):
    """examples/corpus/nlp/05_gpt.psk LayerNorm: (x - mu) / sqrt(var + eps) * g + b.
    `keep`: the training entry keeps the values the gradient reads
    (x - mu, sqrt(var + eps), the normalized x), so they reach memory."""
    with b.func("LayerNorm.apply"):
        return _layernorm_in(b, x, g, bias, keep, tag)


def _layernorm_in(b: Builder, x, g, bias, keep: bool, tag: str):
    mu = b.mean(x, "model", name=f"{tag}.mu")
    if not keep:
        # fusion groups (crates/presk-core/src/fusion.rs:138) join only
        # values of one result type: {x - mu, ^2} and {x - mu, /, *, +} of
        # [batch, seq, model], {var + eps, sqrt} of [batch, seq]
        sq = b.fused([("sub", [("in", 0), ("in", 1)]), ("pow2", [("step", 0)])], [x, mu], x)
        var = b.mean(sq, "model")
        sd = b.fused([("add", [("in", 0), ("in", 1)]), ("sqrt", [("step", 0)])], [var, "eps"], var, name=f"{tag}.sd")
        return b.fused([("sub", [("in", 0), ("in", 1)]), ("div", [("step", 0), ("in", 2)]), ("mul", [("step", 1), ("in", 3)]),
                        ("add", [("step", 2), ("in", 4)])], [x, mu, sd, g, bias], x), {}
    xm = b.binary("sub", x, mu, name=f"{tag}.xm")
    sq = b.unary("pow2", xm, name=f"{tag}.sq")
    var = b.mean(sq, "model", name=f"{tag}.var")
    sd = b.fused([("add", [("in", 0), ("in", 1)]), ("sqrt", [("step", 0)])], [var, "eps"], var, name=f"{tag}.sd")
    xh = b.binary("div", xm, sd, name=f"{tag}.xh")
    y = b.fused([("mul", [("in", 0), ("in", 1)]), ("add", [("step", 0), ("in", 2)])], [xh, g, bias], xh, name=f"{tag}.y")
    return y, {"x": x, "xm": xm, "sq": sq, "sd": sd, "xh": xh, "g": g, "b": bias}


def _layernorm_vjp(b: Builder, saved, dy, tag):
    """The LayerNorm's reverse mode (rules.rs: add, mul, div, sqrt, pow(2),
    mean, sub), cotangents added where a value has two consumers.  Returns dx,
    dg, dbias."""
    with b.func("LayerNorm.apply.vjp"):
        return _layernorm_vjp_in(b, saved, dy, tag)


def _layernorm_vjp_in(b: Builder, saved, dy, tag):
    xm, sd, xh, g = saved["xm"], saved["sd"], saved["xh"], saved["g"]
    db = b.sum_to(dy, saved["b"], name=f"{tag}.dbias")                      # add: sum_to to b's axes
    dg = b.sum_to(b.binary("mul", dy, xh), g, name=f"{tag}.dg")            # mul by g: ct * xh, to g's axes
    dxh = b.binary("mul", dy, g)                                            # ct * g
    # div xh = xm / sd: d xm = ct / sd;  d sd = sum_to(-(ct * xh) / sd)
    dsd = b.sum_to(b.fused([("mul", [("in", 0), ("in", 1)]), ("div", [("step", 0), ("in", 2)]), ("neg", [("step", 1)])],
                           [dxh, xh, sd], dxh), sd)
    # sqrt: d(var + eps) = dsd / (2 * sd)
    dvar = b.fused([("mul", [("in", 0), ("in", 1)]), ("div", [("in", 2), ("step", 0)])], ["two", sd, dsd], sd)
    # mean: d sq = mean_vjp(dvar);  pow(2): d xm += d sq * (2 * xm); plus dxh / sd
    dsq = b.mean_vjp(dvar, saved["sq"], "model")
    dxm = b.fused([("div", [("in", 0), ("in", 1)]), ("pow1", [("in", 3)]), ("mul", [("in", 2), ("step", 1)]),
                   ("mul", [("in", 4), ("step", 2)]), ("add", [("step", 0), ("step", 3)])],
                  [dxh, sd, "two", xm, dsq], xm)
    # sub xm = x - mu: d x = dxm;  d mu = sum_to(-dxm);  mean: d x += mean_vjp(d mu)
    dmu = b.sum_to(b.unary("neg", dxm), f"{tag}.mu")
    dx2 = b.mean_vjp(dmu, saved["x"], "model")
    dx = b.binary("add", dxm, dx2)
    return dx, dg, db


def site_keys(s: GptShape, step_key: bytes) -> list:
    """The keys of the program's dropout sites in slot order, derived from the
    step's key as 05_gpt.psk splits it: (ke, kb) = split_key(k) in GPT.apply
    (ke the embedding's); each block of the fold then splits the carried key
    three times, (katt, k1), (kres, k2), (kff, k3), and carries k3 on."""
    from . import keys
    ke, kb = keys.split(step_key, 2)
    out = [ke]
    for _ in range(s.L):
        katt, k1 = keys.split(kb, 2)
        kres, k2 = keys.split(k1, 2)
        kff, kb = keys.split(k2, 2)
        out += [katt, kres, kff]
    return out


def build(s: GptShape, dtype: str = "f32", train: bool = True, mode=None, realize=None, dropout: float = 0.0,
          step_key: bytes | None = None, optimizer: bool = False) -> tuple:
    """The program of config 3 (`train=False`: loss only) or config 4.
    Returns (program, builder, names) with names["loss"] and, for training,
    names["grads"][param] = buffer of its gradient.  `realize`: a
    Realization giving each site its storage type (else `dtype` everywhere);
    parameters are held at rest in its `params` types (else f32) and every
    kernel reads its inputs converted at its edge.  `dropout`: the rate of
    the program's dropout sites (the course's 0.2) with training masks drawn
    from `step_key` (Key::from_seed(0) by default); 0 leaves them out (x * 1,
    the configs' reading)."""
    from . import hip, keys
    tag = dtype if realize is None else "mixed"
    p = Program(f"gpt-{'step' if train else 'forward'}-{tag}", mode=hip.FAST if mode is None else mode)
    b = Builder(p, dtype, realize)
    if realize is not None:
        b.params_of(opt_leaves(s), params_layout(s)[1], param_shapes(s))
        for name in ("eps", "scale", "two", "one"):
            p.input_types[name] = "f32"
    for name, axes in param_shapes(s).items():
        b.input(name, axes)
    # each block parameter's layers held in one stacked buffer, as `params GPT`
    # stores them (a reference checkpoint's leaf decodes straight into it)
    for n, (axes, members) in opt_leaves(s).items():
        if members is None:
            continue
        tys = {p.input_types.get(m, dtype if realize is None else None) for m in members}
        if len(tys) == 1 and None not in tys and not tys & {"int8", "int4"}:
            count = 1
            for a in axes[1:]:
                count *= a.len
            p.stack(n, members, tys.pop(), count)
    b.input("ids", A(("batch", s.B), ("seq", s.T)), "idx")
    b.input("y", A(("batch", s.B), ("seq", s.T)), "idx")
    b.input("eps", A())
    b.input("scale", A())       # sqrt(HD : R), the attention scores' divisor
    b.input("two", A())         # real(2) of pow(2)'s and sqrt's adjoints
    b.input("one", A())         # the loss's cotangent
    drop = dropout > 0.0
    if drop:
        p.set_keys(site_keys(s, step_key if step_key is not None else keys.from_seed(0)))
    mask = b.causal_mask(s.T, "mask")
    pos_ids = b.positions(s.T, "pos_ids")
    with b.func("Embedding.apply"):
        te = b.embed("tok", "ids", name="te")
        pe = b.embed("pos", pos_ids, name="pe")
        x = b.binary("add", te, pe, name="h0")
    m_emb = None
    if drop:
        # dropout(0.2, ke, h0) = h0 * mask; h0 also gives the mask its shape,
        # so it reaches memory and the mul is a kernel of its own
        with b.func("MiniGPT.apply"):
            m_emb = b.dropout_mask(x, 0, dropout, name="m.emb")
            x0 = x
            x = b.binary("mul", x0, m_emb, name="h0d")
    saved = []
    H, HD = s.H, s.HD
    lbl_q = ["batch", "heads", "seq", "hd"]
    lbl_k = ["batch", "heads", "seq2", "hd"]
    lbl_s = ["batch", "heads", "seq", "seq2"]
    for l in range(s.L):
        pr = f"b{l}."
        xn1, ln1 = _layernorm(b, x, pr + "ln1.g", pr + "ln1.b", train, f"b{l}.ln1")
        with b.func("SelfAttention.apply"):
            q = b.dot(xn1, pr + "wq", pr + "wq.b", name=pr + "q")
            k = b.dot(xn1, pr + "wk", pr + "wk.b", name=pr + "k")
            v = b.dot(xn1, pr + "wv", pr + "wv.b", name=pr + "v")
            qh = b.split_heads(q, H, HD, name=pr + "qh")
            kh = b.split_heads(k, H, HD, name=pr + "kh")
            vh = b.split_heads(v, H, HD, name=pr + "vh")
            sc = b.ein(qh, kh, lbl_q, lbl_k, lbl_s, name=pr + "scores")
            sc2 = b.binary("div", sc, "scale", name=pr + "scaled")
            a = b.masked_softmax(sc2, mask, "seq2", name=pr + "probs")
            ad, ma = a, None
            if drop:
                ma = b.dropout_mask(a, 1 + 3 * l, dropout, name=pr + "m.att")
                ad = b.binary("mul", a, ma, name=pr + "probs_d")
            o = b.ein(ad, vh, lbl_s, lbl_k, lbl_q, name=pr + "o")
            om = b.merge_heads(o, H, HD, name=pr + "om")
            ao = b.dot(om, pr + "wo", pr + "wo.b", name=pr + "ao")
        mr = mf = None
        with b.func("Block.apply"):
            if drop:
                # x + dropout(kres, ao): {ao * m, x + .} one group (ao also
                # shapes the mask, so it reaches memory)
                mr = b.dropout_mask(ao, 2 + 3 * l, dropout, name=pr + "m.res")
                h = b.fused([("mul", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("step", 0)])], [ao, mr, x], x, name=pr + "h")
            else:
                h = b.binary("add", x, ao, name=pr + "h")
        xn2, ln2 = _layernorm(b, h, pr + "ln2.g", pr + "ln2.b", train, f"b{l}.ln2")
        with b.func("MLP.apply"):
            u = b.dot(xn2, pr + "up", pr + "up.b", name=pr + "u")
            g = b.unary("gelu", u, name=pr + "g")
            dn = b.dot(g, pr + "down", pr + "down.b", name=pr + "dn")
        with b.func("Block.apply"):
            if drop:
                mf = b.dropout_mask(dn, 3 + 3 * l, dropout, name=pr + "m.ff")
                xo = b.fused([("mul", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("step", 0)])], [dn, mf, h], h, name=pr + "xo")
            else:
                xo = b.binary("add", h, dn, name=pr + "xo")
        saved.append(dict(x=x, xn1=xn1, ln1=ln1, qh=qh, kh=kh, vh=vh, a=a, ad=ad, ma=ma, mr=mr, mf=mf, om=om, h=h,
                          xn2=xn2, ln2=ln2, u=u, g=g))
        x = xo
    xf, lnf = _layernorm(b, x, "lnf.g", "lnf.b", train, "lnf")
    logits = b.dot(xf, "head", name="logits")
    ce = b.cross_entropy(logits, "y", name="ce")
    loss = b.mean_all(ce, name="loss")
    names = {"loss": loss, "logits": logits, "grads": {}}
    if not train:
        return p, b, names
    G = names["grads"]
    # ---- reverse mode -------------------------------------------------------
    with b.func("MiniGPT.apply.vjp"):
        dce = b.mean_vjp("one", ce, None)
        dlogits = b.cross_entropy_vjp(logits, "y", dce)
        dxf = b.dot_vjp_l(dlogits, "head")
        G["head"] = b.dot_vjp_r(xf, dlogits, name="d.head")
    dx, G["lnf.g"], G["lnf.b"] = _layernorm_vjp(b, lnf, dxf, "lnf")
    for l in reversed(range(s.L)):
        pr, sv = f"b{l}.", saved[l]
        # xo = h + dn (* mf): dn's cotangent is dx (* mf, mul's rule)
        ddn = dx if sv["mf"] is None else b.binary("mul", dx, sv["mf"])
        with b.func("MLP.apply.vjp"):
            dg_ = b.dot_vjp_l(ddn, pr + "down")
            G[pr + "down"] = b.dot_vjp_r(sv["g"], ddn, name="d." + pr + "down")
            G[pr + "down.b"] = b.sum_to(ddn, pr + "down.b", name="d." + pr + "down.b")
            du = b.fused([("gelu_deriv", [("in", 1)]), ("mul", [("in", 0), ("step", 0)])], [dg_, sv["u"]], sv["u"])
            dxn2 = b.dot_vjp_l(du, pr + "up")
            G[pr + "up"] = b.dot_vjp_r(sv["xn2"], du, name="d." + pr + "up")
            G[pr + "up.b"] = b.sum_to(du, pr + "up.b", name="d." + pr + "up.b")
        dh_ln, G[pr + "ln2.g"], G[pr + "ln2.b"] = _layernorm_vjp(b, sv["ln2"], dxn2, f"b{l}.ln2")
        with b.func("Block.apply.vjp"):
            dh = b.binary("add", dx, dh_ln)
        # h = x + ao (* mr)
        dao = dh if sv["mr"] is None else b.binary("mul", dh, sv["mr"])
        with b.func("SelfAttention.apply.vjp"):
            dom = b.dot_vjp_l(dao, pr + "wo")
            G[pr + "wo"] = b.dot_vjp_r(sv["om"], dao, name="d." + pr + "wo")
            G[pr + "wo.b"] = b.sum_to(dao, pr + "wo.b", name="d." + pr + "wo.b")
            do = b.split_heads(dom, H, HD)
            da = b.ein(do, sv["vh"], lbl_q, lbl_k, lbl_s, like=sv["a"])
            dvh = b.ein(do, sv["ad"], lbl_q, lbl_s, lbl_k, like=sv["vh"])
            # the dropped weights ad = a * ma: a's cotangent da * ma
            if sv["ma"] is not None:
                da = b.binary("mul", da, sv["ma"])
            # softmax: a * (da - broadcast(sum(da * a)))
            t = b.binary("mul", da, sv["a"])
            ssum = b.sum(t, "seq2")
            sb = b.broadcast_like(ssum, da)
            dsc2 = b.fused([("sub", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("step", 0)])], [da, sb, sv["a"]], da)
            dsc = b.binary("div", dsc2, "scale")
            dqh = b.ein(dsc, sv["kh"], lbl_s, lbl_k, lbl_q, like=sv["qh"])
            dkh = b.ein(dsc, sv["qh"], lbl_s, lbl_q, lbl_k, like=sv["kh"])
            dq, dk, dv = b.merge_heads(dqh, H, HD), b.merge_heads(dkh, H, HD), b.merge_heads(dvh, H, HD)
            dxq = b.dot_vjp_l(dq, pr + "wq")
            dxk = b.dot_vjp_l(dk, pr + "wk")
            dxv = b.dot_vjp_l(dv, pr + "wv")
            for w, dw in (("wq", dq), ("wk", dk), ("wv", dv)):
                G[pr + w] = b.dot_vjp_r(sv["xn1"], dw, name="d." + pr + w)
                G[pr + w + ".b"] = b.sum_to(dw, pr + w + ".b", name="d." + pr + w + ".b")
            dxn1 = b.fused([("add", [("in", 0), ("in", 1)]), ("add", [("step", 0), ("in", 2)])], [dxq, dxk, dxv], dxq)
        dx_ln, G[pr + "ln1.g"], G[pr + "ln1.b"] = _layernorm_vjp(b, sv["ln1"], dxn1, f"b{l}.ln1")
        with b.func("Block.apply.vjp"):
            dx = b.binary("add", dh, dx_ln)
    # h0 = te + pe (* m.emb): te's cotangent dx (* m.emb); pe's sum_to over the batch
    if m_emb is not None:
        with b.func("MiniGPT.apply.vjp"):
            dx = b.binary("mul", dx, m_emb)
    with b.func("Embedding.apply.vjp"):
        G["tok"] = b.embed_vjp("tok", "ids", dx, name="d.tok")
        dpe = b.sum_to(dx, pe)
        G["pos"] = b.embed_vjp("pos", pos_ids, dpe, name="d.pos")
    if optimizer:
        # the training run's step: `value_vjp` then `adamw.step` (crates/presk-train/src/step.rs)
        if realize is not None:
            raise ValueError("E7005: the optimizer step is built for one storage type (no mixed realization)")
        names["adamw"] = adamw(b, s, G)
    return p, b, names


# ---- the optimizer step (adamw.step) ------------------------------------------------

# 05_gpt.psk's `optimizer adamw` (examples/corpus/nlp/05_gpt.psk:112-117); eps
# takes its default (crates/presk-core/src/lower/optim.rs:58)
ADAMW = {"lr": "3e-4", "beta1": "0.9", "beta2": "0.95", "eps": "1e-8", "weight_decay": "0.1", "grad_clip": "1.0",
         "warmup": 100}
# the literals the step reads, as the host makes them: f64 text, then one
# rounding into the storage type (`Real` of an f64, host.rs's `scalar`)
_OPT_LITS = {"opt.one": "1", "opt.b1": "beta1", "opt.b2": "beta2", "opt.eps": "eps", "opt.wd": "weight_decay",
             "opt.clip": "grad_clip", "opt.tiny": "1e-6", "opt.lr": "lr", "opt.w": "warmup", "opt.half": "0.5"}
# at most this many scalars a kernel sums (a kernel reads at most 24 buffers)
_SUM_CHUNK = 21


# Block's leaves in its tree's order: Block has no params of its own; its
# uses attn (wq, wk, wv, wo: Linear's params w, b), ff (up, down), ln1 and
# ln2 (LayerNorm's params gamma, beta) (05_gpt.psk:28-71)
_BLOCK_LEAVES = ["wq", "wq.b", "wk", "wk.b", "wv", "wv.b", "wo", "wo.b", "up", "up.b", "down", "down.b",
                 "ln1.g", "ln1.b", "ln2.g", "ln2.b"]


def opt_leaves(s: GptShape) -> dict:
    """The leaves adamw.step walks, in order: the tree `params GPT` denotes,
    a module's own params first and then its uses, each in declaration order
    (crates/presk-types/src/elab/mod.rs:191-203): tok, pos, head, then
    blocks, then lnf (05_gpt.psk:80-85); the blocks' leaves stacked along a
    leading layer axis (`stack{L}(Block)`, ParamsTree::Stacked,
    crates/presk-types/src/ty.rs:131-136).  name -> (axes, the per-layer
    parameters it stacks, or None)."""
    ps = param_shapes(s)
    out = {n: (ps[n], None) for n in ("tok", "pos", "head")}
    for r in _BLOCK_LEAVES:
        out["blocks." + r] = ([L.Axis("layer", s.L)] + ps["b0." + r], [f"b{l}.{r}" for l in range(s.L)])
    for n in ("lnf.g", "lnf.b"):
        out[n] = (ps[n], None)
    return out


# a leaf of Block as `params GPT` names it -> its name here
_BLOCK_PATHS = {"wq": "attn.wq.w", "wq.b": "attn.wq.b", "wk": "attn.wk.w", "wk.b": "attn.wk.b",
                "wv": "attn.wv.w", "wv.b": "attn.wv.b", "wo": "attn.wo.w", "wo.b": "attn.wo.b",
                "up": "ff.up.w", "up.b": "ff.up.b", "down": "ff.down.w", "down.b": "ff.down.b",
                "ln1.g": "ln1.γ", "ln1.b": "ln1.β", "ln2.g": "ln2.γ", "ln2.b": "ln2.β"}


def params_layout(s: GptShape):
    """(layout, rename) of a `params GPT` file: the tree in its leaf order
    (opt_leaves), Block's leaves stacked, and the program buffer of each
    leaf's dotted path (`blocks.attn.wq.w` -> the stacked `blocks.wq`)."""
    from .pskd import Layout, Leaf
    rename = {"blocks." + path: "blocks." + r for r, path in _BLOCK_PATHS.items()}
    rename.update({"lnf.γ": "lnf.g", "lnf.β": "lnf.b"})
    back = {v: k for k, v in rename.items()}
    pairs = [(back.get(n, n), Leaf(tuple(a.len for a in axes))) for n, (axes, _) in opt_leaves(s).items()]
    return Layout.from_paths(pairs), rename


def optimizer_inputs(s: GptShape, t: int, total: int, hyper: dict = ADAMW) -> dict:
    """The step's host inputs: the moments of every leaf at zero
    (adamw.init), the literals, pi (PrimOp::Pi, f64 pi rounded once), and the
    step counters t and total (`Real` of a nat)."""
    out = {}
    for name, (axes, _) in opt_leaves(s).items():
        n = 1
        for a in axes:
            n *= a.len
        out["m." + name] = np.zeros(n, np.float32)
        out["v." + name] = np.zeros(n, np.float32)
    # the host's literals are f64s, each rounded once into its storage type
    for k, v in _OPT_LITS.items():
        out[k] = np.array([float(hyper.get(v, v))], np.float64)
    out["opt.pi"] = np.array([math.pi], np.float64)
    out["opt.t"] = np.array([float(t)], np.float64)
    out["opt.total"] = np.array([float(total)], np.float64)
    return out


# adamw.step's and adamw.lr's bodies as crates/presk-core/src/lower/optim.rs
# emits them (optim.rs:160-237, 240-310: the clipped step and the cosine
# schedule), each `let` (name, op, operands, type): `p` the parameter tree,
# `s` a scalar.  A literal is `Real` of an f64 (not elementwise): the
# program's 0-dim input of that value (`lit:<input>`); `Real` of a nat the
# same (`real:<input>`); `pi` is PrimOp::Pi (not elementwise); `g`, `m`, `v`
# and `theta` are the function's parameters; `lr` the call of adamw.lr.
def _step_lets():
    F = Let
    return [
        F("n2", "sum_squares", ["g"], "s"),
        F("norm", "sqrt", ["n2"], "s"), F("tiny", "lit:opt.tiny", [], "s"), F("denom", "add", ["norm", "tiny"], "s"),
        F("clip", "lit:opt.clip", [], "s"), F("coef", "div", ["clip", "denom"], "s"),
        F("one_f", "lit:opt.one", [], "s"), F("fd", "sub", ["one_f", "coef"], "s"), F("fr", "relu", ["fd"], "s"),
        F("factor", "sub", ["one_f", "fr"], "s"),
        F("gc", "mul", ["g", "factor"], "p"),
        F("one", "lit:opt.one", [], "s"), F("b1", "lit:opt.b1", [], "s"), F("b2", "lit:opt.b2", [], "s"),
        F("omb1", "sub", ["one", "b1"], "s"), F("omb2", "sub", ["one", "b2"], "s"),
        F("ma", "mul", ["m", "b1"], "p"), F("mc", "mul", ["gc", "omb1"], "p"), F("m2", "add", ["ma", "mc"], "p"),
        F("va", "mul", ["v", "b2"], "p"), F("gg", "mul", ["gc", "gc"], "p"), F("vc", "mul", ["gg", "omb2"], "p"),
        F("v2", "add", ["va", "vc"], "p"),
        F("tr", "real:opt.t", [], "s"),
        F("lnb1", "log", ["b1"], "s"), F("tl1", "mul", ["tr", "lnb1"], "s"), F("pw1", "exp", ["tl1"], "s"),
        F("bc1", "sub", ["one", "pw1"], "s"),
        F("lnb2", "log", ["b2"], "s"), F("tl2", "mul", ["tr", "lnb2"], "s"), F("pw2", "exp", ["tl2"], "s"),
        F("bc2", "sub", ["one", "pw2"], "s"),
        F("mhat", "div", ["m2", "bc1"], "p"), F("vhat", "div", ["v2", "bc2"], "p"), F("sq", "sqrt", ["vhat"], "p"),
        F("eps", "lit:opt.eps", [], "s"), F("den", "add", ["sq", "eps"], "p"), F("upd", "div", ["mhat", "den"], "p"),
        F("lam", "lit:opt.wd", [], "s"), F("decay", "mul", ["theta", "lam"], "p"), F("dir", "add", ["upd", "decay"], "p"),
        F("lr", "call", [], "s"), F("scaled", "mul", ["dir", "lr"], "p"), F("theta2", "sub", ["theta", "scaled"], "p"),
        F("s2", "tuple", ["m2", "v2"], "t"), F("res", "tuple", ["theta2", "s2"], "t"),
    ], "res"


def _lr_lets():
    F = Let
    return [
        F("base", "lit:opt.lr", [], "s"), F("tr", "real:opt.t", [], "s"), F("totr", "real:opt.total", [], "s"),
        F("w", "lit:opt.w", [], "s"), F("one", "lit:opt.one", [], "s"),
        F("q", "div", ["tr", "w"], "s"), F("one_w", "lit:opt.one", [], "s"), F("wd", "sub", ["one_w", "q"], "s"),
        F("wr", "relu", ["wd"], "s"), F("warm", "sub", ["one_w", "wr"], "s"),
        F("num", "sub", ["tr", "w"], "s"), F("den0", "sub", ["totr", "w"], "s"), F("den1", "sub", ["den0", "one"], "s"),
        F("den2", "relu", ["den1"], "s"), F("den", "add", ["den2", "one"], "s"), F("q2", "div", ["num", "den"], "s"),
        F("r2", "relu", ["q2"], "s"), F("one_p", "lit:opt.one", [], "s"), F("pd", "sub", ["one_p", "r2"], "s"),
        F("pr", "relu", ["pd"], "s"), F("p", "sub", ["one_p", "pr"], "s"),
        F("pi", "lit:opt.pi", [], "s"), F("x", "mul", ["pi", "p"], "s"), F("c", "cos", ["x"], "s"),
        F("s", "add", ["one", "c"], "s"), F("half", "lit:opt.half", [], "s"), F("dec", "mul", ["s", "half"], "s"),
        F("f", "mul", ["warm", "dec"], "s"), F("lr", "mul", ["base", "f"], "s"),
    ], "lr"


def _emit_body(b: Builder, lets, result, env: dict, leaves: list, tag: str, special=None):
    """Runs a body's `let`s as the kernel host runs them: each fusion group
    (presk_amd.fusion.plan) one nest at its root -- a group of the
    parameter tree's type mapped over the tree's leaves, one nest a leaf
    (fusion.rs:104-110) -- every other elementwise `let` a nest of its own,
    the rest by `special(let, env)`.  `env` maps a value to its buffer, or
    for a tree to {leaf: buffer}.  Returns `env`."""
    groups = FU.plan(lets, result)
    interior = {m for g in groups.values() for m in g.members if m != g.root}

    def arg(v, leaf):
        x = env[v]
        return x[leaf] if isinstance(x, dict) else x

    for lt in lets:
        if lt.var in interior:
            continue
        if lt.op.startswith("lit:") or lt.op.startswith("real:"):
            env[lt.var] = lt.op.split(":", 1)[1]
            continue
        if lt.op not in FU.ELEMENTWISE:
            if special is not None:
                special(lt, env)
            continue
        g = groups.get(lt.var)
        steps = g.steps if g else [(lt.op, [("in", i) for i in range(len(lt.args))])]
        ins = g.inputs if g else list(dict.fromkeys(lt.args))
        if not g:
            steps = [(lt.op, [("in", ins.index(a)) for a in lt.args])]
        single = g is None and len(steps) == 1
        if lt.ty == "p":
            out = {}
            for n in leaves:
                srcs = [arg(v, n) for v in ins]
                name = f"{tag}.{lt.var}.{n}"
                if single and len(lt.args) == 2:
                    out[n] = b.binary(lt.op, arg(lt.args[0], n), arg(lt.args[1], n), name=name)
                elif single:
                    out[n] = b.unary(lt.op, arg(lt.args[0], n), name=name)
                else:
                    out[n] = b.fused(steps, srcs, n, name=name)
            env[lt.var] = out
        else:
            srcs = [arg(v, None) for v in ins]
            name = f"{tag}.{lt.var}"
            if single and len(lt.args) == 2:
                env[lt.var] = b.binary(lt.op, arg(lt.args[0], None), arg(lt.args[1], None), name=name)
            elif single:
                env[lt.var] = b.unary(lt.op, arg(lt.args[0], None), name=name)
            else:
                env[lt.var] = b.fused(steps, srcs, "opt.one", name=name)
    return env


def adamw(b: Builder, s: GptShape, grads: dict, hyper: dict = ADAMW) -> dict:
    """adamw.step and adamw.lr (crates/presk-core/src/lower/optim.rs:160-310)
    over the parameters and their gradients, as the kernel host runs them:
    the bodies' fusion groups (crates/presk-core/src/fusion.rs:138, restated
    in presk_amd/fusion.py) each one nest -- values inside a group in f32,
    the arithmetic type, only its root stored in the storage type -- a group
    over the parameter tree mapped leaf by leaf (host.rs:1732-1787), the
    scalars as 0-dim kernels; SumSquares as one `sum_squares` nest a leaf
    added in f64 on the host in leaf order (host.rs:1571-1587) -- here f64
    kernels over the leaves' scalars read through the edge conversion to
    f64, their result read back through the one to the storage type
    (`scalar`'s rounding).  The leaves are `opt_leaves`: a stacked leaf's
    parameters and gradients are its layers' buffers, held one after
    another in one buffer (Program.stack), as StackParams lays them out.
    Returns {leaf: (theta', m', v')}."""
    leaves = opt_leaves(s)
    names = list(leaves)
    grads = dict(grads)
    for n, (axes, members) in leaves.items():
        if members is None:
            continue
        count = 1
        for a in axes[1:]:
            count *= a.len
        if b.p.bufs.views.get(members[0], ("",))[0] != n:
            raise ValueError(f"E7005: the layers of `{n}` are not held in one buffer")
        b.p.stack("d." + n, [grads[m] for m in members], b.dt, count)
        b.input(n, axes)
        grads[n] = b.input("d." + n, axes)
    for k in list(_OPT_LITS) + ["opt.pi", "opt.t", "opt.total"]:
        b.input(k, A())
    for n in names:
        b.input("m." + n, b.axes[n])
        b.input("v." + n, b.axes[n])
    with b.func("adamw.lr"):
        lets, res = _lr_lets()
        lr = _emit_body(b, lets, res, {}, names, "opt.lr")["lr"]

    def special(lt, env):
        if lt.op == "sum_squares":
            # the global norm's square: each leaf's sum of squares, added in
            # f64 in leaf order, at most _SUM_CHUNK a kernel
            ss = [b._prim(lambda dt, g=grads[n]: L.sum_squares([b.op(g)], dt), [grads[n]], f"opt.ss.{n}") for n in names]
            acc = None
            for i in range(0, len(ss), _SUM_CHUNK):
                part = ss[i:i + _SUM_CHUNK]
                ins = ([acc] if acc else []) + part
                steps = [("add", [("in", 0), ("in", 1)])] + [("add", [("step", k), ("in", k + 2)]) for k in range(len(ins) - 2)]
                acc = b._out(L.fused(steps, [b.op(x) for x in ins], [], "f64"), ins, f"opt.n2.{i // _SUM_CHUNK}")
            env[lt.var] = acc
        elif lt.op == "call":
            env[lt.var] = lr
    with b.func("adamw.step"):
        lets, res = _step_lets()
        env = {"g": {n: grads[n] for n in names}, "m": {n: "m." + n for n in names},
               "v": {n: "v." + n for n in names}, "theta": {n: n for n in names}}
        env = _emit_body(b, lets, res, env, names, "opt", special)
    return {n: (env["theta2"][n], env["m2"][n], env["v2"][n]) for n in names}


def host_inputs(s: GptShape, seed: int = 2) -> dict:
    """The seeded synthetic inputs: parameters, token ids and targets uniform
    over the vocabulary, and the scalar constants."""
    host = init_params(s, seed)
    rng = np.random.default_rng(seed + 100)
    host["ids"] = rng.integers(0, s.V, size=(s.B, s.T), dtype=np.int64)
    host["y"] = rng.integers(0, s.V, size=(s.B, s.T), dtype=np.int64)
    host["eps"] = np.array([1e-5], np.float64)
    host["scale"] = np.array([math.sqrt(float(s.HD))], np.float64)
    host["two"] = np.array([2.0], np.float64)
    host["one"] = np.array([1.0], np.float64)
    return host


def contraction_flops(s: GptShape, train: bool) -> float:
    """Algorithmic contraction flops of one call: 2*prod(outer)*I*J*K summed
    over the nests (the forward's, and the gradient's two per contraction)."""
    N = s.B * s.T
    per_layer = 2 * N * s.D * s.D * 4 + 2 * N * s.D * 4 * s.D * 2 + 2 * s.B * s.H * s.T * s.T * s.HD * 2
    fwd = s.L * per_layer + 2 * N * s.D * s.V
    return fwd * 3 if train else fwd
