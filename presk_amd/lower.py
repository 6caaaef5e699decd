"""The loop nests the reference's lowering emits for the primitives of the
measured configurations, as PSK-Kernel text.

A restatement of crates/presk-kernel/src/lower.rs at the default layout
(crates/presk-rt/src/layout.rs:155-199) and the declared orders: each function
names the reference function it follows.  The text is what the reference's
`impl Display for Kernel` prints (crates/presk-kernel/src/ir.rs:495-595), so
the same string is what a Rust host would hand the executor across the C ABI.
Pinned by tests/test_lower.py against the reference's own snapshots
(conformance__linear_kernels.snap, kernels__linear_c.snap).

Expressions and statements are built as text directly.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from decimal import Decimal

SQRT_2 = math.sqrt(2.0)
SQRT_2PI = math.sqrt(2.0 * math.pi)


@dataclass(frozen=True)
class Axis:
    name: str | None
    len: int


def ax(*spec) -> list:
    """ax(("batch", 4), 3) -> [Axis("batch", 4), Axis(None, 3)]."""
    return [Axis(s[0], s[1]) if isinstance(s, tuple) else Axis(None, s) for s in spec]


@dataclass
class Operand:
    axes: list
    kind: str = "real"          # "real", "idx", or a narrower storage type name (BufKind::Wide)


NATURAL_LANES = {"f64": 2, "f32": 4, "bf16": 1, "f16": 1, "e8m15": 1}   # Dtype::natural_lanes (lib.rs:139-141)


def num(x) -> str:
    """An f64 as Rust's Display prints it: shortest round-trip digits, never
    an exponent, no trailing `.0`."""
    x = float(x)
    if x != x:
        return "NaN"
    if x in (float("inf"), float("-inf")):
        return "inf" if x > 0 else "-inf"
    if x == int(x) and abs(x) < 1e16:
        s = str(int(x))
        return "-0" if x == 0 and math.copysign(1, x) < 0 else s
    r = repr(x)
    if "e" in r or "E" in r:
        r = format(Decimal(r), "f")
    return r


# ----- text builders (ir.rs:513-584) ---------------------------------------------

def bin_(op, a, b):
    return f"({a} {op} {b})"


def un(f, a):
    return f"{f}({a})"


def cmp(op, a, b):
    return f"({a} {op} {b})"


def select(c, a, b):
    return f"select({c}, {a}, {b})"


def load(b, ix):
    return f"%{b}[{', '.join(ix)}]"


def iv(v):
    return f"i{v}"


def sv(v):
    return f"s{v}"


def For(var, bound, body):
    return ("for", var, bound, body)


def Set(var, value):
    return ("line", f"s{var} = {value}")


def SetI(var, value):
    return ("line", f"n{var} = {value}")


def SetL(var, value):
    return ("line", f"i{var} = {value}")


def VSet(var, value):
    return ("line", f"v{var} = {value}")


def Store(buf, ix, value):
    return ("line", f"%{buf}[{', '.join(ix)}] = {value}")


def VStore(buf, ix, value):
    return ("line", f"%{buf}[{', '.join(ix)}] <v= {value}")


def If(cond, body):
    return ("if", cond, body)


def _show(body, depth, out):
    pad = "  " * depth
    for s in body:
        if s[0] == "for":
            out.append(f"{pad}for i{s[1]} in 0..{s[2]} {{")
            _show(s[3], depth + 1, out)
            out.append(pad + "}")
        elif s[0] == "if":
            out.append(f"{pad}if {s[1]} {{")
            _show(s[2], depth + 1, out)
            out.append(pad + "}")
        else:
            out.append(pad + s[1])


class B:
    """Variable numbering (lower.rs:74-113)."""

    def __init__(self):
        self.nloops = self.nreal = self.nint = self.nvec = 0
        self.lanes = 1

    def iv(self):
        self.nloops += 1
        return self.nloops - 1

    def sv(self):
        self.nreal += 1
        return self.nreal - 1

    def si(self):
        self.nint += 1
        return self.nint - 1

    def vv(self, lanes):
        self.lanes = lanes
        self.nvec += 1
        return self.nvec - 1

    def loops(self, dims):
        return [self.iv() for _ in dims]


def nest(ivs, dims, body):
    b = body
    for v, d in reversed(list(zip(ivs, dims))):
        b = [For(v, d, b)]
    return b


@dataclass
class Lowered:
    """A lowered primitive: its text, storage type, lane width and output axes."""
    text: str
    dtype: str
    lanes: int
    out_axes: list
    out_kind: str = "real"
    name: str = ""


def _spec(axes, ty):
    parts = [f"{a.name}: {a.len}" if a.name is not None else str(a.len) for a in axes]
    return f"{ty}[{', '.join(parts)}]"


def _buf_ty(kind, dtype):
    if kind == "idx":
        return "i64"
    if kind == "real":
        return dtype
    return kind  # Wide(d)


def kernel(name, dtype, ins, out_axes, out_kind, bd, body) -> Lowered:
    specs = ", ".join(f"%{i} : {_spec(o.axes, _buf_ty(o.kind, dtype))}" for i, o in enumerate(ins))
    out = [f"kernel {name} ({specs}) -> %{len(ins)} : {_spec(out_axes, _buf_ty(out_kind, dtype))} {{"]
    _show(body, 1, out)
    out.append("}")
    return Lowered("\n".join(out) + "\n", dtype, bd.lanes, list(out_axes), out_kind, name)


def dims(axes):
    return [a.len for a in axes]


def ivs(v):
    return [iv(x) for x in v]


# ----- alignment (lower.rs:37-69) --------------------------------------------------

def align(src, target):
    if len(src) > len(target):
        return None
    off = len(target) - len(src)
    if all(a.len == t.len and (a.name is None or t.name is None or a.name == t.name) for a, t in zip(src, target[off:])):
        return list(range(off, len(target)))
    out = []
    for a in src:
        if a.name is None:
            return None
        p = next((i for i, t in enumerate(target) if t.name == a.name and t.len == a.len), None)
        if p is None:
            return None
        out.append(p)
    return out


def result_axes(a, b):
    long, short = (a, b) if len(a) >= len(b) else (b, a)
    m = align(short, long)
    if m is None:
        raise ValueError("cannot broadcast")
    out = list(long)
    for i, p in enumerate(m):
        if out[p].name is None:
            out[p] = Axis(short[i].name, out[p].len)
    return out


# ----- elementwise (lower.rs:167-371) ------------------------------------------------

def gelu(x):
    phi = bin_("/", bin_("+", num(1), un("erf", bin_("/", x, num(SQRT_2)))), num(2))
    return bin_("*", x, phi)


def gelu_deriv(x):
    phi = bin_("/", bin_("+", num(1), un("erf", bin_("/", x, num(SQRT_2)))), num(2))
    dens = bin_("/", un("exp", bin_("/", un("neg", bin_("*", x, x)), num(2))), num(SQRT_2PI))
    return bin_("+", phi, bin_("*", x, dens))


def binary_expr(op, x, y):
    if op in ("add", "sub", "mul", "div"):
        return bin_({"add": "+", "sub": "-", "mul": "*", "div": "/"}[op], x, y)
    if op == "max":
        return select(cmp(">", x, y), x, y)
    if op == "min":
        return select(cmp("<", x, y), x, y)
    raise ValueError(op)


def unary_expr(op, x):
    if op in ("neg", "exp", "log", "tanh", "sqrt", "sin", "cos", "abs"):
        return un(op, x)
    if op == "gelu":
        return gelu(x)
    if op == "gelu_deriv":
        return gelu_deriv(x)
    if op == "relu":
        return select(cmp("<", x, num(0)), num(0), x)
    if op == "heaviside":
        return select(cmp(">", x, num(0)), num(1), num(0))
    if op == "sign":
        return select(cmp("<", x, num(0)), num(-1), select(cmp(">", x, num(0)), num(1), num(0)))
    if op == "sigmoid":
        return bin_("/", num(1), bin_("+", num(1), un("exp", un("neg", x))))
    if op.startswith("pow"):
        n = int(op[3:])
        if n == 0:
            return num(1)
        e = x
        for _ in range(1, n):
            e = bin_("*", e, x)
        return e
    if op == "real":
        return x
    raise ValueError(op)


def elementwise_binary(op, ins, dtype) -> Lowered:
    """lower.rs:309-322."""
    a, b = ins
    out = result_axes(a.axes, b.axes)
    ma, mb = align(a.axes, out), align(b.axes, out)
    bd = B()
    v = bd.loops(dims(out))
    value = binary_expr(op, load(0, [iv(v[p]) for p in ma]), load(1, [iv(v[p]) for p in mb]))
    return kernel(op, dtype, ins, out, "real", bd, nest(v, dims(out), [Store(2, ivs(v), value)]))


def unary(op, ins, dtype) -> Lowered:
    """lower.rs:362-371."""
    a = ins[0]
    bd = B()
    v = bd.loops(dims(a.axes))
    x = f"real({load(0, ivs(v))})" if a.kind == "idx" else load(0, ivs(v))
    # PrimOp::name (crates/presk-core/src/ir.rs:345-420): `pow n`, `gelu'`
    name = f"pow {op[3:]}" if op.startswith("pow") else {"gelu_deriv": "gelu'"}.get(op, op)
    return kernel(name, dtype, ins, a.axes, "real", bd, nest(v, dims(a.axes), [Store(1, ivs(v), unary_expr(op, x))]))


def fused(steps, ins, out, dtype) -> Lowered:
    """lower.rs:328-360: `steps` are (op, [src...]) with src ('in', k) or ('step', k)."""
    bd = B()
    v = bd.loops(dims(out))
    idx = []
    for o in ins:
        m = align(o.axes, out)
        if m is None:
            raise ValueError("fused: operand does not broadcast")
        idx.append([iv(v[p]) for p in m])
    vals = []
    for op, args in steps:
        a = []
        for src, k in args:
            if src == "in":
                a.append(f"real({load(k, idx[k])})" if ins[k].kind == "idx" else load(k, idx[k]))
            else:
                a.append(vals[k])
        vals.append(unary_expr(op, a[0]) if len(a) == 1 else binary_expr(op, a[0], a[1]))
    body = nest(v, dims(out), [Store(len(ins), ivs(v), vals[-1])])
    return kernel(f"fused {len(steps)} steps", dtype, ins, out, "real", bd, body)


# ----- contractions (lower.rs:695-1219) --------------------------------------------------

@dataclass
class Contraction:
    name: str
    out: list
    outer: list
    i: int
    j: int
    k: int
    ks: list
    x_index: list     # slots: ('o', p), 'I', 'J', 'K'
    w_index: list
    dot: bool
    nt: bool
    inline_x: bool


def contraction_of(op, ins, ein_operands=None, ein_output=None):
    """`Contraction::of` (lower.rs:695-784), under an exact order."""
    if op == "dot":
        x, w = ins[0].axes, ins[1].axes
        if len(w) != 2 or len(x) < 2 or x[-1].len != w[0].len:
            return None
        p = len(x) - 2
        return Contraction("dot", x[:p + 1] + [w[1]], [a.len for a in x[:p]], x[p].len, w[1].len, w[0].len, [w[0].len],
                           [("o", q) for q in range(p)] + ["I", "K"], ["K", "J"], True, False, False)
    if op == "dot_vjp_l":
        ct, b = ins[0].axes, ins[1].axes
        if len(b) != 2 or len(ct) < 2 or ct[-1].len != b[1].len:
            return None
        p = len(ct) - 2
        return Contraction("dot_vjp_l", ct[:p + 1] + [b[0]], [a.len for a in ct[:p]], ct[p].len, b[0].len, b[1].len,
                           [b[1].len], [("o", q) for q in range(p)] + ["I", "K"], ["J", "K"], False, True, True)
    if op == "dot_vjp_r":
        a, ct = ins[0].axes, ins[1].axes
        lead = len(a) - 1
        if lead <= 0 or len(ct) != len(a) or any(x.len != y.len for x, y in zip(a[:lead], ct[:lead])):
            return None
        ks = [x.len for x in a[:lead]]
        return Contraction("dot_vjp_r", [a[lead], ct[lead]], [], a[lead].len, ct[lead].len, math.prod(ks), ks,
                           ["K", "I"], ["K", "J"], False, False, True)
    if op == "ein":
        n = len(ein_output)
        A, Bn = ein_operands
        if n < 2 or len(A) != n or len(Bn) != n or len(ins[0].axes) != n or len(ins[1].axes) != n:
            return None
        outer, i, j = ein_output[:n - 2], ein_output[n - 2], ein_output[n - 1]
        ks = [x for x in A if x not in ein_output]
        if len(ks) != 1:
            return None
        k = ks[0]

        def slot(x, own, own_slot):
            if x == k:
                return "K"
            if x == own:
                return own_slot
            return ("o", outer.index(x)) if x in outer else None

        xi = [slot(x, i, "I") for x in A]
        wi = [slot(x, j, "J") for x in Bn]
        if None in xi or None in wi:
            return None
        lx = lambda s: ins[0].axes[xi.index(s)].len
        lw = lambda s: ins[1].axes[wi.index(s)].len
        outer_len = [lx(("o", p)) for p in range(len(outer))]
        ni, nj, nk = lx("I"), lw("J"), lx("K")
        out = [Axis(o, l) for o, l in zip(outer, outer_len)] + [Axis(i, ni), Axis(j, nj)]
        return Contraction(f"ein[{', '.join(ein_output)}]", out, outer_len, ni, nj, nk, [nk], xi, wi, False, wi[-1] == "K", False)
    return None


def _blocked(v, n, t):
    """`blocked` (lower.rs:874-877)."""
    return iv(v) if n == 1 else bin_("+", bin_("*", iv(v), str(n)), str(t))


def _slots(idx, outer, i, j, k):
    out = []
    for s in idx:
        if isinstance(s, tuple):
            out.append(iv(outer[s[1]]))
        elif s == "I":
            out.append(i)
        elif s == "J":
            out.append(j)
        else:
            out.extend(k)
    return out


def default_layout(c: Contraction, dtype):
    """`Layout::resolve` for a contraction (layout.rs:162-184)."""
    accum_is_storage = dtype in ("f32", "f64")
    if c.dot and c.j % 8 != 0 and accum_is_storage:
        return {"form": "row", "lanes": 1}
    tile = (1, 8) if c.dot and c.j % 8 == 0 else (1, 1)
    width = NATURAL_LANES[dtype]
    lanes = width if tile[1] % width == 0 and not c.nt else 1
    return {"form": "tiled", "tile": tile, "lanes": lanes}


def emit_contraction(c: Contraction, dtype, ins, layout=None, epilogue=None) -> Lowered:
    """`emit_contraction_with` (lower.rs:906-1139) at a layout without a
    k-block, and `row_wise` (lower.rs:1184-1219).  `epilogue` = (first, out
    axes) adds the last input (lower.rs:846-864)."""
    layout = layout or default_layout(c, dtype)
    bias = None
    if epilogue is not None:
        first, eout = epilogue
        bias = align(ins[2].axes, eout)
    name = c.name + ("+add" if epilogue is not None else "")
    out_axes = epilogue[1] if epilogue is not None else c.out
    add = (lambda s, b: bin_("+", s, b) if epilogue[0] else bin_("+", b, s)) if epilogue is not None else None
    buf_out = len(ins)
    if layout["form"] == "row":
        bd = B()
        rows = c.outer + [c.i]
        ov = bd.loops(rows)
        kv = bd.loops(c.ks)
        jv, acc = bd.iv(), bd.sv()
        outer, ivv = ov[:-1], iv(ov[-1])

        def cix(j):
            return ivs(ov) + [iv(j)]
        zero = For(jv, c.j, [Store(buf_out, cix(jv), num(0))])
        kx = ivs(kv)
        xix = _slots(c.x_index, outer, ivv, "0", kx)
        wix = _slots(c.w_index, outer, ivv, iv(jv), kx)
        sweep = For(jv, c.j, [Store(buf_out, cix(jv), bin_("+", load(buf_out, cix(jv)), bin_("*", sv(acc), load(1, wix))))])
        body = [zero] + nest(kv, c.ks, [Set(acc, load(0, xix)), sweep])
        if epilogue is not None:
            rank = len(c.out)
            bix = [iv(jv) if p + 1 == rank else iv(ov[p]) for p in bias]
            body.append(For(jv, c.j, [Store(buf_out, cix(jv), add(load(buf_out, cix(jv)), load(2, bix)))]))
        return kernel(name, dtype, ins, out_axes, "real", bd, nest(ov, rows, body))
    mi, nj = layout["tile"]
    lanes = layout["lanes"]
    if c.i % mi or c.j % nj or nj % lanes:
        raise ValueError("tile does not fit")
    bd = B()
    ov = bd.loops(c.outer)
    vi, vj = bd.iv(), bd.iv()
    kv = bd.loops(c.ks)
    kx = ivs(kv)
    vector = lanes > 1
    cols = nj // lanes
    inline = c.inline_x and mi == 1 and nj == 1
    fresh = (lambda: bd.vv(lanes)) if vector else bd.sv
    accs = [[fresh() for _ in range(cols)] for _ in range(mi)]
    xs = [] if inline else [bd.sv() for _ in range(mi)]
    ws = [fresh() for _ in range(cols)] if mi > 1 else []

    def ix(r):
        return _blocked(vi, mi, r)

    def jx(g):
        return _blocked(vj, nj, g * lanes)

    def out_ix(r, g):
        return ivs(ov) + [ix(r), jx(g)]

    def x_at(r):
        return _slots(c.x_index, ov, ix(r), "0", kx)

    def w_at(g):
        return _slots(c.w_index, ov, "0", jx(g), kx)

    def x_of(r):
        return load(0, x_at(r)) if inline else sv(xs[r])

    micro = [Set(x, load(0, x_at(r))) for r, x in enumerate(xs)]
    for g, w in enumerate(ws):
        micro.append(VSet(w, f"{load(1, w_at(g))}<v>") if vector else Set(w, load(1, w_at(g))))
    for r, row in enumerate(accs):
        for g, a in enumerate(row):
            if g < len(ws):
                wv = f"v{ws[g]}" if vector else sv(ws[g])
            else:
                wv = f"{load(1, w_at(g))}<v>" if vector else load(1, w_at(g))
            if vector:
                micro.append(VSet(a, f"(v{a} + (splat({x_of(r)}) * {wv})<v>)<v>"))
            else:
                micro.append(Set(a, bin_("+", sv(a), bin_("*", x_of(r), wv))))
    init, store = [], []
    for r, row in enumerate(accs):
        for g, a in enumerate(row):
            init.append(VSet(a, f"splat({num(0)})") if vector else Set(a, num(0)))
            store.append(VStore(buf_out, out_ix(r, g), f"v{a}") if vector else Store(buf_out, out_ix(r, g), sv(a)))
    narrow = dtype not in ("f32", "f64")
    epi = []
    if epilogue is not None:
        rank = len(c.out)
        for r, row in enumerate(accs):
            for g, a in enumerate(row):
                at = [iv(ov[p]) if p + 2 < rank else (ix(r) if p + 2 == rank else jx(g)) for p in bias]
                if vector:
                    q = [k for k, p in enumerate(bias) if p + 1 == rank]
                    b = f"{load(2, at)}<v>" if q and q[0] + 1 == len(bias) else f"splat({load(2, at)})"
                    s, t = (f"v{a}", b) if epilogue[0] else (b, f"v{a}")
                    epi.append(VSet(a, f"({s} + {t})<v>"))
                elif narrow:
                    epi.append(Store(buf_out, out_ix(r, g), add(load(buf_out, out_ix(r, g)), load(2, at))))
                else:
                    epi.append(Set(a, add(sv(a), load(2, at))))
    over_k = nest(kv, c.ks, micro)
    tile_body = init + over_k + ([] if narrow else epi) + store + (epi if narrow else [])
    body = [For(vi, c.i // mi, [For(vj, c.j // nj, tile_body)])]
    return kernel(name, dtype, ins, out_axes, "real", bd, nest(ov, c.outer, body))


def exact_order(order) -> bool:
    """`ReductionOrder::is_exact` (crates/presk-rt/src/lib.rs:273-275): the
    sequential and blocked orders keep the index order of every addition;
    `("interleaved", n)` and `("chunked", c)` reassociate."""
    return not order or order[0] not in ("interleaved", "chunked")


def order_of(o) -> tuple | None:
    """A realization's `order` ({"kind": ..., "partials"/"size"/"width": n},
    lib.rs:249-270) as this module's tuple; None for the exact ones."""
    if o is None:
        return None
    kind = o.get("kind") if isinstance(o, dict) else o[0]
    if kind in ("sequential", "blocked"):
        return None
    if kind == "interleaved":
        return ("interleaved", int(o["partials"] if isinstance(o, dict) else o[1]))
    if kind == "chunked":
        return ("chunked", int(o["size"] if isinstance(o, dict) else o[1]))
    raise ValueError(f"E7001: the reduction order `{kind}`")


def _chunked_only(order):
    """lower.rs:299-303: the derivatives of `dot` and `ein` take a chunked
    order; any other is the sequential one for them."""
    return order if order and order[0] == "chunked" else None


def contraction_ordered(name, dtype, ins, out, outer_dims, inner_dims, index_x, index_y, order) -> Lowered:
    """lower.rs:384-475: one output element a thread of the nest, its terms
    x[index_x] * w[index_y] summed under `order`:
    - ("interleaved", n), one summed axis that n divides, n >= 2: n partial
      accumulators, the t-th summing terms cb*n + t in order, added left to
      right at the end;
    - ("chunked", c), one summed axis: chunks of c consecutive terms each
      summed from zero, the chunk sums added to the total in order from
      zero, the last chunk what is left;
    - otherwise every term in index order into one accumulator."""
    if order and order[0] == "interleaved" and len(inner_dims) == 1 and order[1] >= 2 and inner_dims[0] % order[1] == 0:
        n = order[1]
        chunks = inner_dims[0] // n
        bd = B()
        ov = bd.loops(outer_dims)
        cb = bd.iv()
        terms = [bd.iv() for _ in range(n)]
        accs = [bd.sv() for _ in range(n)]
        inner = []
        for t in range(n):
            inner.append(SetL(terms[t], bin_("+", bin_("*", iv(cb), str(n)), str(t))))
            inner.append(Set(accs[t], bin_("+", sv(accs[t]), bin_("*", load(0, index_x(ov, [terms[t]])),
                                                                  load(1, index_y(ov, [terms[t]]))))))
        body = [Set(a, num(0)) for a in accs]
        body.append(For(cb, chunks, inner))
        total = sv(accs[0])
        for a in accs[1:]:
            total = bin_("+", total, sv(a))
        body.append(Store(2, ivs(ov), total))
        return kernel(name, dtype, ins, out, "real", bd, nest(ov, outer_dims, body))
    if order and order[0] == "chunked":
        size = order[1]
        if len(inner_dims) != 1:
            raise ValueError(f"{name}: the order chunked({size}) sums one summed axis in chunks, and this sum runs over "
                             f"{len(inner_dims)} axes")
        if size == 0:
            raise ValueError(f"{name}: the order chunked(0) has no chunk")
        k = inner_dims[0]
        bd = B()
        ov = bd.loops(outer_dims)
        cb, t, kvv = bd.iv(), bd.iv(), bd.iv()
        acc, part = bd.sv(), bd.sv()
        term = bin_("*", load(0, index_x(ov, [kvv])), load(1, index_y(ov, [kvv])))

        def chunk(start, length):
            return [Set(part, num(0)),
                    For(t, length, [SetL(kvv, bin_("+", start, iv(t))), Set(part, bin_("+", sv(part), term))]),
                    Set(acc, bin_("+", sv(acc), sv(part)))]
        body = [Set(acc, num(0))]
        if k // size > 0:
            body.append(For(cb, k // size, chunk(bin_("*", iv(cb), str(size)), size)))
        if k % size > 0:
            body.extend(chunk(str(k // size * size), k % size))
        body.append(Store(2, ivs(ov), sv(acc)))
        return kernel(name, dtype, ins, out, "real", bd, nest(ov, outer_dims, body))
    bd = B()
    ov = bd.loops(outer_dims)
    cv = bd.loops(inner_dims)
    acc = bd.sv()
    inner = nest(cv, inner_dims, [Set(acc, bin_("+", sv(acc), bin_("*", load(0, index_x(ov, cv)), load(1, index_y(ov, cv)))))])
    body = [Set(acc, num(0))] + inner + [Store(2, ivs(ov), sv(acc))]
    return kernel(name, dtype, ins, out, "real", bd, nest(ov, outer_dims, body))


def _dot_ordered(ins, dtype, order) -> Lowered:
    """lower.rs:481-510: `x[..., K] . w[K, rest...]` as `contraction_ordered`."""
    x, w = ins[0], ins[1]
    k = x.axes[-1].len
    lead = len(x.axes) - 1
    out = list(x.axes[:lead]) + list(w.axes[1:])
    return contraction_ordered("dot", dtype, ins, out, dims(out), [k],
                               lambda ov, cv: [iv(v) for v in ov[:lead]] + [iv(cv[0])],
                               lambda ov, cv: [iv(cv[0])] + [iv(v) for v in ov[lead:]], order)


def _dot_vjp_l_ordered(ins, dtype, order) -> Lowered:
    """lower.rs:516-546: `ct[..., N...] . b[K, N...]^T -> [..., K]`."""
    ct, b = ins[0], ins[1]
    k = len(b.axes) - 1
    lead = len(ct.axes) - k
    out = list(ct.axes[:lead]) + [b.axes[0]]
    return contraction_ordered("dot_vjp_l", dtype, ins, out, dims(out), [a.len for a in b.axes[1:]],
                               lambda ov, cv: [iv(v) for v in ov[:lead]] + [iv(v) for v in cv],
                               lambda ov, cv: [iv(ov[lead])] + [iv(v) for v in cv], order)


def _dot_vjp_r_ordered(ins, dtype, order) -> Lowered:
    """lower.rs:552-584: `a[..., K], ct[..., N...] -> [K, N...]` summed over
    the leading axes."""
    a, ct = ins[0], ins[1]
    lead = len(a.axes) - 1
    out = [a.axes[lead]] + list(ct.axes[lead:])
    return contraction_ordered("dot_vjp_r", dtype, ins, out, dims(out), [x.len for x in a.axes[:lead]],
                               lambda ov, cv: [iv(v) for v in cv] + [iv(ov[0])],
                               lambda ov, cv: [iv(v) for v in cv] + [iv(v) for v in ov[1:]], order)


def dot(ins, dtype, order=None, layout=None, epilogue=None) -> Lowered:
    """`lower_planned` for `dot` (lower.rs:250-266): a contraction nest
    (Contraction::of, only under an exact order) in its layout, else
    `dot`'s ordered form."""
    c = contraction_of("dot", ins) if exact_order(order) else None
    if c is None:
        if epilogue is not None:
            raise ValueError("dot: an epilogue is a contraction nest's")
        return _dot_ordered(ins, dtype, order)
    return emit_contraction(c, dtype, ins, layout, epilogue)


def dot_vjp_l(ins, dtype, order=None) -> Lowered:
    c = contraction_of("dot_vjp_l", ins) if exact_order(order) else None
    if c is None:
        return _dot_vjp_l_ordered(ins, dtype, _chunked_only(order))
    return emit_contraction(c, dtype, ins)


def dot_vjp_r(ins, dtype, order=None) -> Lowered:
    c = contraction_of("dot_vjp_r", ins) if exact_order(order) else None
    if c is None:
        return _dot_vjp_r_ordered(ins, dtype, _chunked_only(order))
    return emit_contraction(c, dtype, ins)


def ein(ins, operands, output, dtype, order=None) -> Lowered:
    """`ein` (lower.rs:586-636): a contraction nest where the operands' roles
    fit one (`Contraction::of`, under an exact order), else under a chunked
    order the chunked contraction of two operands over one summed axis, else
    the generic many-operand form: one accumulator per output element over
    the summed axes, its term `(1 * x0) * x1 ...`."""
    c = contraction_of("ein", ins, operands, output) if exact_order(order) else None
    if c is not None:
        return emit_contraction(c, dtype, ins)
    order = _chunked_only(order)
    names = []
    for t, ns in zip(ins, operands):
        for a, n in zip(t.axes, ns):
            if not any(m == n for m, _ in names):
                names.append((n, a.len))
    contracted = [(n, l) for n, l in names if n not in output]
    out = [Axis(o, next(l for n, l in names if n == o)) for o in output]
    name = f"ein[{', '.join(output)}]"
    if order is not None:
        if len(ins) != 2 or len(contracted) != 1:
            raise ValueError(f"{name}: the order chunked({order[1]}) sums the product of two operands over one summed "
                             f"axis in chunks, and this one has {len(ins)} operands and {len(contracted)} summed axes")
        pos = [[output.index(n) if n in output else None for n in ns] for ns in operands]

        def at(ix, ov, cv):
            return [iv(cv[0] if p is None else ov[p]) for p in ix]
        return contraction_ordered(name, dtype, ins, out, dims(out), [contracted[0][1]],
                                   lambda ov, cv: at(pos[0], ov, cv), lambda ov, cv: at(pos[1], ov, cv), order)
    allv = list(output) + [n for n, _ in contracted]
    bd = B()
    ov = bd.loops(dims(out))
    cv = bd.loops([l for _, l in contracted])
    all_v = ov + cv
    acc = bd.sv()
    prod = num(1)
    for i, ns in enumerate(operands):
        ix = [iv(all_v[allv.index(n)]) for n in ns]
        prod = bin_("*", prod, load(i, ix))
    inner = nest(cv, [l for _, l in contracted], [Set(acc, bin_("+", sv(acc), prod))])
    body = [Set(acc, num(0))] + inner + [Store(len(ins), ivs(ov), sv(acc))]
    return kernel(f"ein[{', '.join(output)}]", dtype, ins, out, "real", bd, nest(ov, dims(out), body))


# ----- reductions (lower.rs:1221-1419, 1670-1703) ------------------------------------------

def _axis_pos(axes, name):
    for i, a in enumerate(axes):
        if a.name == name:
            return i
    raise ValueError(f"no axis {name}")


def reduce_all(op, ins, dtype) -> Lowered:
    """lower.rs:1221-1233 (SumAll/MeanAll: the kernels `sum` and `mean`,
    PrimOp::name, crates/presk-core/src/ir.rs:371-372); `op` "sum"/"mean"
    ("sum_all"/"mean_all" name the same)."""
    op = {"sum_all": "sum", "mean_all": "mean"}.get(op, op)
    t = ins[0]
    bd = B()
    v = bd.loops(dims(t.axes))
    acc = bd.sv()
    body = [Set(acc, num(0))] + nest(v, dims(t.axes), [Set(acc, bin_("+", sv(acc), load(0, ivs(v))))])
    n = math.prod(dims(t.axes))
    value = bin_("/", sv(acc), num(n)) if op == "mean" else sv(acc)
    body.append(Store(1, [], value))
    return kernel(op, dtype, ins, [], "real", bd, body)


def reduce_axis(op, axis, ins, dtype) -> Lowered:
    """lower.rs:1239-1255 (`sum axis a`/`mean axis a`)."""
    t = ins[0]
    p = _axis_pos(t.axes, axis)
    out = list(t.axes)
    n = out.pop(p).len
    bd = B()
    ov = bd.loops(dims(out))
    k = bd.iv()
    acc = bd.sv()
    full = ivs(ov)
    full.insert(p, iv(k))
    body = [Set(acc, num(0)), For(k, n, [Set(acc, bin_("+", sv(acc), load(0, full)))])]
    value = bin_("/", sv(acc), num(n)) if op == "mean" else sv(acc)
    body.append(Store(1, ivs(ov), value))
    return kernel(f"{op} axis {axis}", dtype, ins, out, "real", bd, nest(ov, dims(out), body))


def _softmax_rows(bd, buf, axes, p):
    outer = list(axes)
    n = outer.pop(p).len
    ov = bd.loops(dims(outer))
    k = bd.iv()
    m, z = bd.sv(), bd.sv()

    def full(i):
        v = ivs(ov)
        v.insert(p, i)
        return v
    stmts = [Set(m, load(buf, full("0"))),
             For(k, n, [If(cmp(">", load(buf, full(iv(k))), sv(m)), [Set(m, load(buf, full(iv(k))))])]),
             Set(z, num(0)),
             For(k, n, [Set(z, bin_("+", sv(z), un("exp", bin_("-", load(buf, full(iv(k))), sv(m)))))])]
    return ov, m, z, stmts, k, n, outer


def softmax(axis, ins, dtype) -> Lowered:
    """lower.rs:1296-1311 (three passes)."""
    t = ins[0]
    p = _axis_pos(t.axes, axis)
    bd = B()
    ov, m, z, body, k, n, outer = _softmax_rows(bd, 0, t.axes, p)
    full = ivs(ov)
    full.insert(p, iv(k))
    body.append(For(k, n, [Store(1, full, bin_("/", un("exp", bin_("-", load(0, full), sv(m))), sv(z)))]))
    body = [] if n == 0 else nest(ov, dims(outer), body)
    return kernel(f"softmax axis {axis}", dtype, ins, t.axes, "real", bd, body)


def softmax_two_pass(axis, ins, dtype) -> Lowered:
    """lower.rs:1320-1353."""
    t = ins[0]
    p = _axis_pos(t.axes, axis)
    outer = list(t.axes)
    n = outer.pop(p).len
    bd = B()
    ov = bd.loops(dims(outer))
    k = bd.iv()
    m, z, e = bd.sv(), bd.sv(), bd.sv()

    def full(i):
        v = ivs(ov)
        v.insert(p, i)
        return v
    at = full(iv(k))
    body = [Set(m, load(0, full("0"))),
            For(k, n, [If(cmp(">", load(0, at), sv(m)), [Set(m, load(0, at))])]),
            Set(z, num(0)),
            For(k, n, [Set(e, un("exp", bin_("-", load(0, at), sv(m)))), Store(1, at, sv(e)), Set(z, bin_("+", sv(z), sv(e)))]),
            For(k, n, [Store(1, at, bin_("/", load(1, at), sv(z)))])]
    body = [] if n == 0 else nest(ov, dims(outer), body)
    return kernel(f"softmax axis {axis}, two passes", dtype, ins, t.axes, "real", bd, body)


def masked_softmax(axis, ins, dtype, two_passes=False) -> Lowered:
    """lower.rs:1368-1419."""
    t, mk = ins
    p = _axis_pos(t.axes, axis)
    mp = align(mk.axes, t.axes)
    outer = list(t.axes)
    n = outer.pop(p).len
    bd = B()
    ov = bd.loops(dims(outer))
    k = bd.iv()
    mx, z, first, e = bd.sv(), bd.sv(), bd.sv(), bd.sv()
    at = ivs(ov)
    at.insert(p, iv(k))
    x = load(0, at)
    allowed = cmp(">", f"real({load(1, [at[q] for q in mp])})", num(0.5))
    ex = un("exp", bin_("-", x, sv(mx)))
    body = [Set(first, num(1)), Set(mx, num(0)),
            For(k, n, [Set(mx, select(allowed, select(cmp(">", sv(first), num(0.5)), x, select(cmp(">", x, sv(mx)), x, sv(mx))), sv(mx))),
                       Set(first, select(allowed, num(0), sv(first)))]),
            Set(z, num(0))]
    if two_passes:
        body.append(For(k, n, [Set(e, select(allowed, ex, num(0))), Store(2, at, sv(e)), Set(z, bin_("+", sv(z), sv(e)))]))
        body.append(For(k, n, [Store(2, at, select(allowed, bin_("/", load(2, at), sv(z)), num(0)))]))
    else:
        body.append(For(k, n, [Set(z, bin_("+", sv(z), select(allowed, ex, num(0))))]))
        body.append(For(k, n, [Store(2, at, select(allowed, bin_("/", ex, sv(z)), num(0)))]))
    body = [] if n == 0 else nest(ov, dims(outer), body)
    name = f"softmax axis {axis} where" + (", two passes" if two_passes else "")
    return kernel(name, dtype, ins, t.axes, "real", bd, body)


def cross_entropy(ins, dtype) -> Lowered:
    """lower.rs:1459-1471."""
    logits, y = ins
    p = len(logits.axes) - 1
    bd = B()
    ov, m, z, body, _, _, _ = _softmax_rows(bd, 0, logits.axes, p)
    at_y = ivs(ov) + [load(1, ivs(ov))]
    body.append(Store(2, ivs(ov), bin_("-", bin_("+", un("log", sv(z)), sv(m)), load(0, at_y))))
    return kernel("cross_entropy", dtype, ins, y.axes, "real", bd, nest(ov, dims(y.axes), body))


def cross_entropy_vjp(ins, dtype) -> Lowered:
    """lower.rs:1473-1488."""
    logits = ins[0]
    p = len(logits.axes) - 1
    v = logits.axes[p].len
    bd = B()
    ov, m, z, body, _, _, outer = _softmax_rows(bd, 0, logits.axes, p)
    k = bd.iv()
    full = ivs(ov) + [iv(k)]
    onehot = select(cmp("==", f"real({iv(k)})", f"real({load(1, ivs(ov))})"), num(1), num(0))
    sm = bin_("/", un("exp", bin_("-", load(0, full), sv(m))), sv(z))
    body.append(For(k, v, [Store(3, full, bin_("*", bin_("-", sm, onehot), load(2, ivs(ov))))]))
    return kernel("cross_entropy_vjp", dtype, ins, logits.axes, "real", bd, nest(ov, dims(outer), body))


def sum_to(ins, dtype) -> Lowered:
    """lower.rs:1670-1680."""
    x, tmpl = ins
    m = align(tmpl.axes, x.axes)
    bd = B()
    zv = bd.loops(dims(tmpl.axes))
    body = nest(zv, dims(tmpl.axes), [Store(2, ivs(zv), num(0))])
    v = bd.loops(dims(x.axes))
    oix = [iv(v[p]) for p in m]
    body += nest(v, dims(x.axes), [Store(2, oix, bin_("+", load(2, oix), load(0, ivs(v))))])
    return kernel("sum_to", dtype, ins, tmpl.axes, "real", bd, body)


def sum_squares(ins, dtype) -> Lowered:
    """lower.rs:1693-1703."""
    t = ins[0]
    bd = B()
    v = bd.loops(dims(t.axes))
    acc = bd.sv()
    body = [Set(acc, num(0))] + nest(v, dims(t.axes), [Set(acc, bin_("+", sv(acc), bin_("*", load(0, ivs(v)), load(0, ivs(v)))))])
    body.append(Store(1, [], sv(acc)))
    return kernel("sum_squares", dtype, ins, [], "real", bd, body)


def mean_vjp(axis, ins, dtype) -> Lowered:
    """lower.rs:1257-1270."""
    ct, tmpl = ins
    n = math.prod(dims(tmpl.axes)) if axis is None else next((a.len for a in tmpl.axes if a.name == axis), 1)
    m = align(ct.axes, tmpl.axes)
    bd = B()
    v = bd.loops(dims(tmpl.axes))
    body = [Store(2, ivs(v), bin_("/", load(0, [iv(v[p]) for p in m]), num(n)))]
    return kernel("mean_vjp", dtype, ins, tmpl.axes, "real", bd, nest(v, dims(tmpl.axes), body))


def broadcast_like(ins, dtype) -> Lowered:
    """lower.rs:1682-1691."""
    x, tmpl = ins
    m = align(x.axes, tmpl.axes)
    bd = B()
    v = bd.loops(dims(tmpl.axes))
    body = [Store(2, ivs(v), load(0, [iv(v[p]) for p in m]))]
    return kernel("broadcast_like", dtype, ins, tmpl.axes, "real", bd, nest(v, dims(tmpl.axes), body))


# ----- gathers, scatters, permutations (lower.rs:1421-1752) -------------------------------

def embed(ins, dtype) -> Lowered:
    """lower.rs:1421-1437."""
    table, idx = ins
    d = table.axes[1].len
    out = list(idx.axes) + [Axis(None, d)]
    bd = B()
    v = bd.loops(dims(idx.axes))
    j = bd.iv()
    body = [For(j, d, [Store(2, ivs(v) + [iv(j)], load(0, [load(1, ivs(v)), iv(j)]))])]
    return kernel("embed", dtype, ins, out, "real", bd, nest(v, dims(idx.axes), body))


def embed_vjp(ins, dtype) -> Lowered:
    """lower.rs:1444-1457."""
    table, idx, _ct = ins
    d = table.axes[1].len
    bd = B()
    zv = bd.loops(dims(table.axes))
    body = nest(zv, dims(table.axes), [Store(3, ivs(zv), num(0))])
    v = bd.loops(dims(idx.axes))
    j = bd.iv()
    oix = [load(1, ivs(v)), iv(j)]
    body += nest(v, dims(idx.axes), [For(j, d, [Store(3, oix, bin_("+", load(3, oix), load(2, ivs(v) + [iv(j)])))])])
    return kernel("embed_vjp", dtype, ins, table.axes, "real", bd, body)


def split_heads(h, hd, ins, dtype) -> Lowered:
    """lower.rs:1604-1628."""
    t = ins[0]
    r = len(t.axes)
    out = list(t.axes[:r - 2]) + [Axis("heads", h), t.axes[r - 2], Axis("hd", hd)]
    bd = B()
    ov = bd.loops(dims(out))
    n = len(ov)
    ix = ivs(ov[:n - 3]) + [iv(ov[n - 2]), bin_("+", bin_("*", iv(ov[n - 3]), str(hd)), iv(ov[n - 1]))]
    return kernel(f"split_heads {h}x{hd}", dtype, ins, out, "real", bd, nest(ov, dims(out), [Store(1, ivs(ov), load(0, ix))]))


def merge_heads(h, hd, ins, dtype) -> Lowered:
    """lower.rs:1631-1659."""
    t = ins[0]
    r = len(t.axes)
    out = list(t.axes[:r - 3]) + [t.axes[r - 2], Axis("model", h * hd)]
    bd = B()
    ov = bd.loops(dims(out))
    n = len(ov)
    hh, d = bd.iv(), bd.iv()
    oix = ivs(ov[:n - 1]) + [bin_("+", bin_("*", iv(hh), str(hd)), iv(d))]
    ix = ivs(ov[:n - 2]) + [iv(hh), iv(ov[n - 2]), iv(d)]
    body = nest(ov[:n - 1], dims(out[:n - 1]), [For(hh, h, [For(d, hd, [Store(1, oix, load(0, ix))])])])
    return kernel(f"merge_heads {h}x{hd}", dtype, ins, out, "real", bd, body)


def slice_(axis, lo, hi, ins, dtype) -> Lowered:
    """lower.rs:1554-1572: the elements lo..hi of one axis, which keeps its
    name at length hi - lo."""
    t = ins[0]
    p = _axis_pos(t.axes, axis)
    if lo > hi or hi > t.axes[p].len:
        raise ValueError(f"slice {lo}..{hi} outside the axis `{axis}`, of length {t.axes[p].len}")
    out = list(t.axes)
    out[p] = Axis(out[p].name, hi - lo)
    bd = B()
    ov = bd.loops(dims(out))
    src = ivs(ov)
    src[p] = bin_("+", iv(ov[p]), str(lo))
    # an index operand is copied as indices (StoreI of LoadI: the same text)
    kind = "idx" if t.kind == "idx" else "real"
    body = [Store(1, ivs(ov), load(0, src))]
    return kernel(f"slice {axis}: {lo}..{hi}", dtype, ins, out, kind, bd, nest(ov, dims(out), body))


def slice_vjp(axis, lo, hi, ins, dtype) -> Lowered:
    """lower.rs:1574-1590: zeros of the template's shape, the cotangent at
    the elements lo..hi of the axis."""
    tmpl, ct = ins
    p = _axis_pos(tmpl.axes, axis)
    if len(ct.axes) != len(tmpl.axes) or ct.axes[p].len != hi - lo:
        raise ValueError(f"slice_vjp {axis}: {lo}..{hi}: a cotangent of {show(ct.axes)} into {show(tmpl.axes)}")
    bd = B()
    body = _zero_fill(bd, 2, tmpl.axes)
    cv = bd.loops(dims(ct.axes))
    dst = ivs(cv)
    dst[p] = bin_("+", iv(cv[p]), str(lo))
    body += nest(cv, dims(ct.axes), [Store(2, dst, load(1, ivs(cv)))])
    return kernel(f"slice_vjp {axis}: {lo}..{hi}", dtype, ins, tmpl.axes, "real", bd, body)


def _zero_fill(bd, buf, axes):
    """`zero_fill` (lower.rs:1439-1442)."""
    v = bd.loops(dims(axes))
    return nest(v, dims(axes), [Store(buf, ivs(v), num(0))])


def show(axes) -> str:
    """`show` (lower.rs:1754-1760): `[name: len, len]`."""
    return "[" + ", ".join(f"{a.name}: {a.len}" if a.name is not None else str(a.len) for a in axes) + "]"


def argmax(ins, dtype) -> Lowered:
    """lower.rs:1490-1516: the position of the largest element along the
    last axis, seeded from element 0 and moved on `>=`, so that the last of
    equal maxima wins (the interpreter's `max_by`); a NaN never compares, so
    a later NaN is passed over and a NaN at element 0 keeps position 0."""
    t = ins[0]
    if not t.axes:
        raise ValueError("argmax: scalar argument")
    p = len(t.axes) - 1
    v = t.axes[p].len
    out = list(t.axes[:p])
    bd = B()
    ov = bd.loops(dims(out))
    k = bd.iv()
    m = bd.sv()
    best = bd.si()
    full = ivs(ov) + [iv(k)]
    first = ivs(ov) + ["0"]
    body = [Set(m, load(0, first)), SetI(best, "0"),
            For(k, v, [If(cmp(">=", load(0, full), sv(m)), [Set(m, load(0, full)), SetI(best, iv(k))])]),
            Store(1, ivs(ov), f"n{best}")]
    return kernel("argmax", dtype, ins, out, "idx", bd, nest(ov, dims(out), body))


def index_const(axis, index, ins, dtype) -> Lowered:
    """lower.rs:1518-1535: `t[axis: index]` (a negative index counts from the
    end), which drops the axis; for a real and an index tensor."""
    t = ins[0]
    p = _axis_pos(t.axes, axis)
    n = t.axes[p].len
    i = n + index if index < 0 else index
    if i < 0 or i >= n:
        raise ValueError(f"index {index} out of range for axis `{axis}` of length {n}")
    out = list(t.axes[:p]) + list(t.axes[p + 1:])
    bd = B()
    ov = bd.loops(dims(out))
    full = ivs(ov)
    full.insert(p, str(i))
    kind = "idx" if t.kind == "idx" else "real"
    body = [Store(1, ivs(ov), load(0, full))]
    return kernel(f"index {axis}: {index}", dtype, ins, out, kind, bd, nest(ov, dims(out), body))


def scatter_index(axis, index, ins, dtype) -> Lowered:
    """lower.rs:1537-1552: the cotangent of `index`: zeros of the template's
    shape, the cotangent at position `index` of the axis."""
    tmpl, ct = ins
    p = _axis_pos(tmpl.axes, axis)
    n = tmpl.axes[p].len
    i = n + index if index < 0 else index
    bd = B()
    body = _zero_fill(bd, 2, tmpl.axes)
    cv = bd.loops(dims(ct.axes))
    full = ivs(cv)
    full.insert(p, str(i))
    body += nest(cv, dims(ct.axes), [Store(2, full, load(1, ivs(cv)))])
    return kernel(f"scatter_index {axis}: {index}", dtype, ins, tmpl.axes, "real", bd, body)


def one_hot(out, dtype) -> Lowered:
    """lower.rs:1728-1744: 1 where the index equals the position on the new
    trailing axis; `out` is the result's axes, the indices carry all but the
    last."""
    k = len(out) - 1
    idx_axes, v = list(out[:k]), out[k].len
    ins = [Operand(idx_axes, "idx")]
    bd = B()
    lv = bd.loops(dims(idx_axes))
    j = bd.iv()
    hit = cmp("==", f"real({load(0, ivs(lv))})", f"real({iv(j)})")
    body = nest(lv, dims(idx_axes), [For(j, v, [Store(1, ivs(lv) + [iv(j)], select(hit, num(1), num(0)))])])
    return kernel("one_hot", dtype, ins, out, "real", bd, body)


def fill(name, axes, value, dtype) -> Lowered:
    """lower.rs:1746-1752: a constant fill (`zeros`, `ones`)."""
    bd = B()
    v = bd.loops(dims(axes))
    return kernel(name, dtype, [], axes, "real", bd, nest(v, dims(axes), [Store(0, ivs(v), num(value))]))


def pack_panel(c: Contraction, dtype, w: Operand) -> Lowered:
    """lower.rs:1155-1182: operand 1 of an NT contraction copied, in its own
    type, to a panel of axes (the outer axes it carries..., K, J), which the
    contraction then reads as NN; written along J."""
    if len(c.ks) > 1:
        raise ValueError(f"{c.name}: a pack of a sum over several axes")
    carried = [o for o in range(len(c.outer)) if ("o", o) in c.w_index]

    def at(slot):
        return w.axes[c.w_index.index(slot)]

    axes = [at(("o", o)) for o in carried] + [at("K"), at("J")]
    bd = B()
    lv = bd.loops(dims(axes))
    ov = [0] * len(c.outer)
    for n, o in enumerate(carried):
        ov[o] = lv[n]
    p = len(carried)
    src = _slots(c.w_index, ov, "0", iv(lv[p + 1]), [iv(lv[p])])
    body = [Store(1, ivs(lv), load(0, src))]
    return kernel("pack", dtype, [w], axes, "real", bd, nest(lv, dims(axes), body))


def packed(c: Contraction) -> Contraction:
    """`Contraction::packed` (lower.rs:804-809): the same contraction reading
    operand 1 from its NN panel."""
    import dataclasses
    carried = [("o", o) for o in range(len(c.outer)) if ("o", o) in c.w_index]
    return dataclasses.replace(c, w_index=carried + ["K", "J"], nt=False)


def concat(axis, ins, dtype) -> Lowered:
    """lower.rs:1592-1612: `x` into the first part of the axis, `y` into
    the rest, each element written once."""
    x, y = ins
    p, q = _axis_pos(x.axes, axis), _axis_pos(y.axes, axis)
    if not (p == q and len(x.axes) == len(y.axes) and all(k == p or u.len == v.len for k, (u, v) in enumerate(zip(x.axes, y.axes)))):
        raise ValueError(f"concat {axis}: shapes differ off the axis")
    m = x.axes[p].len
    out = list(x.axes)
    out[p] = Axis(out[p].name, m + y.axes[p].len)
    bd = B()
    xv = bd.loops(dims(x.axes))
    body = nest(xv, dims(x.axes), [Store(2, ivs(xv), load(0, ivs(xv)))])
    yv = bd.loops(dims(y.axes))
    dst = ivs(yv)
    dst[p] = bin_("+", iv(yv[p]), str(m))
    body += nest(yv, dims(y.axes), [Store(2, dst, load(1, ivs(yv)))])
    return kernel(f"concat {axis}", dtype, ins, out, "real", bd, body)


def causal_mask(axis, n, dtype) -> Lowered:
    """lower.rs:1717-1726."""
    out = [Axis(axis, n), Axis(f"{axis}2", n)]
    bd = B()
    i, j = bd.iv(), bd.iv()
    below = select(cmp("<=", f"real({iv(j)})", f"real({iv(i)})"), num(1), num(0))
    body = nest([i, j], [n, n], [Store(0, [iv(i), iv(j)], f"int({below})")])
    return kernel(f"causal_mask {axis}", dtype, [], out, "idx", bd, body)


def positions(axis, n, dtype) -> Lowered:
    """lower.rs:1706-1713."""
    out = [Axis(axis, n)]
    bd = B()
    i = bd.iv()
    return kernel(f"positions {axis}", dtype, [], out, "idx", bd, [For(i, n, [Store(0, [iv(i)], iv(i))])])
