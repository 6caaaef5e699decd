"""Config 5: the Llama decoder (examples/coverage/llama.psk) as a program of
the reference's nests -- `Llama.apply`, the logits of a full context, as
`presk serve` recomputes them.

Each function of the program is followed let by let, in its evaluation
order, with the primitives the front end emits for it
(crates/presk-core/src/lower/expr.rs) and the kernels the kernel backend
launches for them (crates/presk-kernel/src/host.rs, lower.rs):

* `split`/`merge` are views of one buffer (host.rs:1510-1536), no launch;
  `p[pair: 0..1]` is a `slice` nest (lower.rs:1554-1572), `concat` its own
  (lower.rs:1592-1612);
* `ein` keeps its operands' axes as the checker labels them, a name shared
  by both operands renamed in the right one when exactly one copy of it
  (`seq` -> `seq2`) dangles (crates/presk-types/src/check/expr.rs:596-640);
* a scalar literal becomes a 0-dim buffer in the site's storage type
  (host.rs:589-591, 1590-1595) and a function of one, `log(real(1e4))`,
  `sqrt(HD : R)`, `-(2 : R)`, a 0-dim kernel (host.rs:1836-1849);
* elementwise lets form fusion groups as crates/presk-core/src/fusion.rs:138
  forms them, per function body: a producer joins its consumer's group when
  it is elementwise, of the same result type (shape included) and read by
  nothing outside the group; `real` of indices is not elementwise.

The configuration's constants differ from the program's in two places, as
the configuration states them: multi-head attention (G = H, the program's
`--const G=32`) and RMSNorm eps 1e-6 (the program's literal is 1e-5).  The
TINY shape keeps G < H so that grouped-query attention's broadcast `ein`s
are exercised.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import lower as L
from .gpt import Builder
from .program import Program

A = L.ax


@dataclass
class LlamaShape:
    V: int = 32000
    D: int = 4096
    H: int = 32
    G: int = 32          # key/value heads (G = H: multi-head attention)
    FF: int = 11008
    L: int = 32
    B: int = 1
    T: int = 2048
    eps: float = 1e-6
    base: float = 1e4    # RoPE's base

    @property
    def HD(self):
        return self.D // self.H

    @property
    def P(self):
        return self.H // self.G


LLAMA_7B = LlamaShape()
TINY = LlamaShape(V=64, D=32, H=4, G=2, FF=48, L=2, B=2, T=8)


def ein_labels(names0, names1, output):
    """The `ein` checker's relabeling of two operands
    (crates/presk-types/src/check/expr.rs:596-640): a name both operands
    carry is renamed in the right operand when exactly one copy of it
    (the name followed by digits) dangles -- in the output and in no
    operand, or in one operand only and not in the output."""
    ops = [list(names0), list(names1)]
    shared = [n for n in ops[0] if n in ops[1]]

    def in_ops(name):
        return sum(1 for o in ops if name in o)

    for n in shared:
        def is_copy(c):
            return len(c) > len(n) and c.startswith(n) and c[len(n):].isdigit()
        dangling = [o for o in output if in_ops(o) == 0 and is_copy(o)]
        for o in ops:
            for a in o:
                if a != n and in_ops(a) == 1 and a not in output and is_copy(a) and a not in dangling:
                    dangling.append(a)
        if len(dangling) == 1:
            ops[1][ops[1].index(n)] = dangling[0]
        elif len(dangling) > 1:
            raise ValueError(f"ambiguous ein: `{n}` could be renamed to {dangling}")
    return ops


def param_shapes(s: LlamaShape) -> dict:
    """name -> axes of every parameter, as llama.psk declares them (a
    `Dense`'s and an `RMSNorm`'s axes are unnamed)."""
    ps = {"tok": A(("vocab", s.V), ("model", s.D))}
    for l in range(s.L):
        p = f"b{l}."
        ps[p + "n1.g"] = A(s.D)
        ps[p + "attn.wq"] = A(("model", s.D), ("qout", s.D))
        ps[p + "attn.wk"] = A(("model", s.D), ("kvout", s.G * s.HD))
        ps[p + "attn.wv"] = A(("model", s.D), ("kvout", s.G * s.HD))
        ps[p + "attn.wo"] = A(("headhd", s.D), ("model", s.D))
        ps[p + "n2.g"] = A(s.D)
        ps[p + "ff.gate"] = A(s.D, s.FF)
        ps[p + "ff.up"] = A(s.D, s.FF)
        ps[p + "ff.down"] = A(s.FF, s.D)
    ps["norm.g"] = A(s.D)
    ps["head"] = A(s.D, s.V)
    return ps


def param_count(s: LlamaShape) -> int:
    n = 0
    for axes in param_shapes(s).values():
        k = 1
        for a in axes:
            k *= a.len
        n += k
    return n


SCALARS = ("two", "hdr", "base", "eps")


def scalar_values(s: LlamaShape) -> dict:
    """The program's literals: `(2 : R)`, `(HD : R)`, `real(1e4)` and the
    RMSNorm eps, each a 0-dim buffer."""
    return {"two": 2.0, "hdr": float(s.HD), "base": float(s.base), "eps": float(s.eps)}


def _rmsnorm(b: Builder, x, g, tag):
    """RMSNorm.apply: `let ms = mean(axis model, x * x); x / sqrt(ms + eps) * g`.
    Groups: `x * x` alone (its consumer is a reduction), {ms + eps, sqrt}
    of type [batch, seq], {div, mul} of type [batch, seq, model]."""
    with b.func("RMSNorm.apply"):
        xx = b.binary("mul", x, x, name=f"{tag}.xx")
        ms = b.mean(xx, "model", name=f"{tag}.ms")
        sd = b.fused([("add", [("in", 0), ("in", 1)]), ("sqrt", [("step", 0)])], [ms, "eps"], ms, name=f"{tag}.sd")
        return b.fused([("div", [("in", 0), ("in", 1)]), ("mul", [("step", 0), ("in", 2)])], [x, sd, g], x, name=f"{tag}.y")


def _frequencies(b: Builder, s: LlamaShape):
    """`exp(-(2 : R) * real(positions(rot: HD/2)) / (HD : R) * log(real(1e4)))`."""
    with b.func("frequencies"):
        n2 = b.unary("neg", "two", name="n2")
        pr = b.positions(s.HD // 2, "pr", axis="rot")
        rr = b.unary("real", pr, name="rr")
        lb = b.unary("log", "base", name="lb")
        return b.fused([("mul", [("in", 0), ("in", 1)]), ("div", [("step", 0), ("in", 2)]),
                        ("mul", [("step", 1), ("in", 3)]), ("exp", [("step", 2)])],
                       [n2, rr, "hdr", lb], rr, name="freq")


def _angles(b: Builder, s: LlamaShape):
    """`ein[seq, rot](real(positions(seq: T)) * frequencies())`."""
    with b.func("angles"):
        ps = b.positions(s.T, "ps", axis="seq")
        rs = b.unary("real", ps, name="rs")
        fr = _frequencies(b, s)
        la, lb = ein_labels(["seq"], ["rot"], ["seq", "rot"])
        return b.ein(rs, fr, la, lb, ["seq", "rot"], name="phi")


def _rope(b: Builder, s: LlamaShape, phi, x, tag):
    """rope: each pair (r, r + HD/2) of a head rotated by t * w_r."""
    with b.func("rope"):
        p = b.split(x, "hd", "pair", 2, "rot", s.HD // 2, name=f"{tag}.p")
        x0 = b.slice(p, "pair", 0, 1, name=f"{tag}.x0")
        x1 = b.slice(p, "pair", 1, 2, name=f"{tag}.x1")
        c = b.unary("cos", phi, name=f"{tag}.c")
        sn = b.unary("sin", phi, name=f"{tag}.s")
        r0 = b.fused([("mul", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("in", 3)]), ("sub", [("step", 0), ("step", 1)])],
                     [x0, c, x1, sn], x0, name=f"{tag}.r0")
        r1 = b.fused([("mul", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("in", 3)]), ("add", [("step", 0), ("step", 1)])],
                     [x1, c, x0, sn], x0, name=f"{tag}.r1")
        cc = b.concat(r0, r1, "pair", name=f"{tag}.cat")
        return b.merge(cc, "pair", "rot", name=f"{tag}.rot")


def _attention(b: Builder, s: LlamaShape, pr, x, mask, phi):
    G, P, HD = s.G, s.P, s.HD
    with b.func("Attention.apply"):
        wq1 = b.split(pr + "attn.wq", "qout", "groups", G, "rest", P * HD)
        wq3 = b.split(wq1, "rest", "per", P, "hd", HD)
        out_q = ["batch", "groups", "per", "seq", "hd"]
        la, lb = ein_labels(["batch", "seq", "model"], ["model", "groups", "per", "hd"], out_q)
        qp = b.ein(x, wq3, la, lb, out_q, name=pr + "qp")
        q = _rope(b, s, phi, qp, pr + "q")
        wk3 = b.split(pr + "attn.wk", "kvout", "groups", G, "hd", HD)
        out_k = ["batch", "groups", "seq", "hd"]
        la, lb = ein_labels(["batch", "seq", "model"], ["model", "groups", "hd"], out_k)
        kp = b.ein(x, wk3, la, lb, out_k, name=pr + "kp")
        k = _rope(b, s, phi, kp, pr + "k")
        vd = b.dot(x, pr + "attn.wv", name=pr + "vd")
        v = b.split(vd, "kvout", "groups", G, "hd", HD, name=pr + "v")
        # q and k as rope's type names them, [..., seq, hd]
        out_s = ["batch", "groups", "per", "seq", "seq2"]
        la, lb = ein_labels(out_q, out_k, out_s)
        sc = b.ein(q, k, la, lb, out_s, name=pr + "scores")
        sq = b.unary("sqrt", "hdr", name=pr + "sqrt_hd")
        sc2 = b.binary("div", sc, sq, name=pr + "scaled")
        a = b.masked_softmax(sc2, mask, "seq2", name=pr + "probs")
        out_o = ["batch", "seq", "groups", "per", "hd"]
        la, lb = ein_labels(out_s, ["batch", "seq", "groups", "hd"], out_o)
        o = b.ein(a, v, la, lb, out_o, name=pr + "o")
        w1 = b.split(pr + "attn.wo", "headhd", "groups", G, "rest", P * HD)
        w2 = b.split(w1, "rest", "per", P, "hd", HD)
        out_y = ["batch", "seq", "model"]
        la, lb = ein_labels(out_o, ["groups", "per", "hd", "model"], out_y)
        return b.ein(o, w2, la, lb, out_y, name=pr + "ao")


def _swiglu(b: Builder, pr, x):
    """`down.apply(silu(gate.apply(x)) * up.apply(x))`; silu's body
    `x * sigmoid(x)` is one group of its own function."""
    with b.func("SwiGLU.apply"):
        with b.func("Dense.apply"):
            g = b.dot(x, pr + "ff.gate", name=pr + "gate")
        with b.func("silu"):
            sg = b.fused([("sigmoid", [("in", 0)]), ("mul", [("in", 0), ("step", 0)])], [g], g, name=pr + "silu")
        with b.func("Dense.apply"):
            u = b.dot(x, pr + "ff.up", name=pr + "up")
        m = b.binary("mul", sg, u, name=pr + "gu")
        with b.func("Dense.apply"):
            return b.dot(m, pr + "ff.down", name=pr + "down")


# a Block leaf here -> its path under `blocks` in `params Llama`: Attention's
# params wq, wk, wv, wo; SwiGLU's uses gate, up, down (Dense's param w);
# RMSNorm's param gamma (llama.psk:29-118)
_BLOCK_PATHS = {"attn.wq": "attn.wq", "attn.wk": "attn.wk", "attn.wv": "attn.wv", "attn.wo": "attn.wo",
                "ff.gate": "ff.gate.w", "ff.up": "ff.up.w", "ff.down": "ff.down.w", "n1.g": "n1.γ", "n2.g": "n2.γ"}


def _count(axes) -> int:
    n = 1
    for a in axes:
        n *= a.len
    return n


def leaves(s: LlamaShape) -> dict:
    """`params Llama`'s leaves in order -- a module's params, then its uses,
    each in declaration order (crates/presk-types/src/elab/mod.rs:191-203):
    tok, head, blocks (`stack{L}(Block)`, each leaf with a leading layer
    axis), norm (llama.psk:120-130).  name -> (axes, the per-layer
    parameters a stacked leaf holds, or None)."""
    ps = param_shapes(s)
    out = {"tok": (ps["tok"], None), "head": (ps["head"], None)}
    for r in _BLOCK_PATHS:
        out["blocks." + r] = ([L.Axis("layer", s.L)] + ps["b0." + r], [f"b{l}.{r}" for l in range(s.L)])
    out["norm.g"] = (ps["norm.g"], None)
    return out


def params_layout(s: LlamaShape):
    """(layout, rename) of a `params Llama` file: its tree (Block's leaves
    stacked) and the program buffer of each leaf's dotted path."""
    from .pskd import Layout, Leaf
    rename = {"blocks." + path: "blocks." + r for r, path in _BLOCK_PATHS.items()}
    rename["norm.γ"] = "norm.g"
    back = {v: k for k, v in rename.items()}
    pairs = [(back.get(n, n), Leaf(tuple(a.len for a in axes))) for n, (axes, _) in leaves(s).items()]
    return Layout.from_paths(pairs), rename


def build(s: LlamaShape, dtype: str = "bf16", mode=None, realize=None) -> tuple:
    """The program of `Llama.apply` (the logits).  Returns (program,
    builder, names) with names["logits"]."""
    from . import hip
    p = Program(f"llama-forward-{dtype if realize is None else 'mixed'}", mode=hip.FAST if mode is None else mode)
    b = Builder(p, dtype, realize)
    b.fn = "Llama.apply"
    if realize is not None:
        b.params_of(leaves(s), params_layout(s)[1], param_shapes(s))
    for name, axes in param_shapes(s).items():
        b.input(name, axes)
    # each block parameter's layers held in one stacked buffer, as `params
    # Llama` stores them (a checkpoint's leaf decodes straight into it)
    for n, (axes, members) in leaves(s).items():
        tys = {p.input_types.get(m, dtype if realize is None else None) for m in members or []}
        if members and len(tys) == 1 and None not in tys and not tys & {"int8", "int4"}:
            p.stack(n, members, tys.pop(), _count(axes[1:]))
    b.input("ids", A(("batch", s.B), ("seq", s.T)), "idx")
    for name in SCALARS:
        b.input(name, A())
    mask = b.causal_mask(s.T, "mask")
    with b.func("Llama.apply"):
        x = b.embed("tok", "ids", name="x0")
    phi = _angles(b, s)
    for l in range(s.L):
        pr = f"b{l}."
        with b.func("Block.apply"):
            h = _rmsnorm(b, x, pr + "n1.g", pr + "n1")
            ao = _attention(b, s, pr, h, mask, phi)
            x2 = b.binary("add", x, ao, name=pr + "x")
            h2 = _rmsnorm(b, x2, pr + "n2.g", pr + "n2")
            f = _swiglu(b, pr, h2)
            x = b.binary("add", x2, f, name=pr + "out")
    xn = _rmsnorm(b, x, "norm.g", "norm")
    with b.func("Llama.apply"):
        logits = b.dot(xn, "head", name="logits")
    return p, b, {"logits": logits}


def host_inputs(s: LlamaShape, seed: int = 5) -> dict:
    """Seeded synthetic inputs at a shape the host can hold: every matrix and
    the token table N(0, 0.02), RMSNorm gains one, ids uniform over the
    vocabulary, and the literals."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, axes in param_shapes(s).items():
        shape = [a.len for a in axes]
        if name.endswith(".g"):
            out[name] = np.ones(shape, np.float32)
        else:
            out[name] = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    out["ids"] = rng.integers(0, s.V, size=(s.B, s.T), dtype=np.int64)
    for k, v in scalar_values(s).items():
        out[k] = np.array([v], np.float64)
    return out


def contraction_flops(s: LlamaShape) -> float:
    """2 * prod(outer) * I * J * K over the forward's contraction nests."""
    N = s.B * s.T
    kv = s.G * s.HD
    per_layer = (2 * N * s.D * s.D * 2          # q projection, output projection
                 + 2 * N * s.D * kv * 2         # k, v
                 + 2 * s.B * s.H * s.T * s.T * s.HD * 2   # scores, values
                 + 2 * N * s.D * s.FF * 3)      # gate, up, down
    return s.L * per_layer + 2 * N * s.D * s.V


def input_specs(p: Program) -> dict:
    """name -> (storage type, element count) of every program input."""
    from .configs import _input_specs
    specs = {}
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, _input_specs(ln.low)):
            specs.setdefault(name, (p.input_types.get(name, ty) if ty != "i64" else ty, count))
    return specs


def load_device_inputs(p: Program, s: LlamaShape, seed: int = 5):
    """Declares every input and fills the parameters in HBM where they live
    (presk_hip_fill_normal: every matrix and the token table N(0, 0.02),
    RMSNorm gains one); the token ids (uniform over the vocabulary) and the
    literals are copied from the host."""
    from . import configs, hip
    specs = input_specs(p)
    lib = hip.lib()
    for i, name in enumerate(param_shapes(s)):
        ty, count = specs[name]
        buf = p.declare(name, ty, max(count, 1))
        mean, std = (1.0, 0.0) if name.endswith(".g") else (0.0, 0.02)
        hip.check(lib.presk_hip_fill_normal(buf.ptr, ty.encode(), count, seed * 1000003 + i, mean, std, None))
    rng = np.random.default_rng(seed)
    host = {"ids": rng.integers(0, s.V, size=(s.B, s.T), dtype=np.int64)}
    host.update({k: np.array([v], np.float64) for k, v in scalar_values(s).items()})
    for name, arr in configs.storage_inputs(p, host).items():
        ty, count = specs[name]
        p.declare(name, ty, max(count, 1))
        p.bufs.upload(name, arr)
    hip.sync()
