"""oracle/kernel_text.py -- TEST INFRASTRUCTURE ONLY (the parity oracle).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything under oracle/.  The product has its own C++ parser.

A reader of PSK-Kernel's textual form, the text `presk dump --stage kernel`
prints (crates/presk-kernel/src/ir.rs:495-595, `impl Display for Kernel`),
into a small tuple AST that oracle/cexec.py turns into C.

The grammar restated from the printer:
  header   kernel NAME (%0 : T[axes], ...) -> %n : T[axes][ arith A product P accum C[ store S]] {
  axes     `name: len` or `len`, comma separated           (ir.rs:497-511 `spec`)
  stmts    one per line, two spaces of indent per level  (ir.rs:561-584)
             for iV in 0..B {   sV = e   nV = e   iV = e   vV = e
             %b[ix] = e         %b[ix] <v= e      if c {   }
  exprs    (ir.rs:513-559) numbers as Rust prints an f64 or an i64, %b[ix],
           %b[ix]<v>, iV sV nV vV, (a OP b), (a OP b)<v>, neg(..) exp(..)
           log tanh sqrt sin cos erf abs, select(c, a, b), real(..), int(..),
           splat(..), comparisons (a < b) (a <= b) (a > b) (a >= b) (a == b).

Pinned by tests/test_oracle_text.py: the reference's own snapshot text
(crates/presk-kernel/tests/snapshots/conformance__linear_kernels.snap and the
kernel comments of crates/presk-export-c/tests/snapshots/kernels__linear_c.snap)
parses and prints back character for character.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

REAL_TYPES = ("f64", "f32", "bf16", "f16", "e8m15")
UNARY = ("neg", "exp", "log", "tanh", "sqrt", "sin", "cos", "erf", "abs")


@dataclass
class Buf:
    ty: str                  # f32 / bf16 / f16 / e8m15 / f64 / i64 / intB/o[..e]
    dims: list
    names: list              # axis names or None

    @property
    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def strides(self) -> list:
        s = [1] * len(self.dims)
        for i in range(len(self.dims) - 2, -1, -1):
            s[i] = s[i + 1] * self.dims[i + 1]
        return s


@dataclass
class Kernel:
    name: str
    inputs: list
    output: Buf
    arith: str | None
    body: list
    text: str = ""
    nloops: int = 0
    nreal: int = 0
    nint: int = 0
    nvec: int = 0
    bufs: list = field(default_factory=list)


# ----- header -------------------------------------------------------------------

def _parse_spec(s: str) -> Buf:
    m = re.fullmatch(r"\s*(\S+?)\[(.*)\]\s*", s)
    if not m:
        raise ValueError(f"bad buffer spec {s!r}")
    ty, axes = m.group(1), m.group(2).strip()
    dims, names = [], []
    if axes:
        for a in axes.split(", "):
            if ": " in a:
                n, d = a.split(": ")
                names.append(n)
                dims.append(int(d))
            else:
                names.append(None)
                dims.append(int(a))
    return Buf(ty, dims, names)


def _split_specs(s: str) -> list:
    """`%0 : f32[a: 4, 3], %1 : f32[3]` -> ['f32[a: 4, 3]', 'f32[3]']."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch == "[":
            depth += 1
        elif ch == "]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    specs = []
    for k, part in enumerate(out):
        part = part.strip()
        pre = f"%{k} : "
        if not part.startswith(pre):
            raise ValueError(f"bad input spec {part!r}")
        specs.append(_parse_spec(part[len(pre):]))
    return specs


# ----- expressions ----------------------------------------------------------------

_TOK = re.compile(r"\s*(<v=|<v>|<=|>=|==|=|\.\.|-?inf|NaN|-?\d+(?:\.\d+)?|%\d+|[A-Za-z_][A-Za-z_0-9]*|[()\[\],<>+\-*/])")


def _tokens(s: str) -> list:
    pos, out = 0, []
    s = s.rstrip()
    while pos < len(s):
        m = _TOK.match(s, pos)
        if not m:
            raise ValueError(f"cannot read {s[pos:]!r}")
        out.append(m.group(1))
        pos = m.end()
    return out


class _P:
    def __init__(self, toks):
        self.t, self.i = toks, 0

    def peek(self):
        return self.t[self.i] if self.i < len(self.t) else None

    def take(self, want=None):
        tok = self.peek()
        if want is not None and tok != want:
            raise ValueError(f"expected {want!r}, found {tok!r} in {' '.join(self.t)}")
        self.i += 1
        return tok

    def index(self):
        self.take("[")
        ix = []
        if self.peek() != "]":
            ix.append(self.expr())
            while self.peek() == ",":
                self.take(",")
                ix.append(self.expr())
        self.take("]")
        return ix

    def expr(self):
        tok = self.take()
        if tok is None:
            raise ValueError("unexpected end of expression")
        if re.fullmatch(r"-?inf|NaN|-?\d+(?:\.\d+)?", tok):
            return ("num", tok)
        if tok.startswith("%"):
            b = int(tok[1:])
            ix = self.index()
            if self.peek() == "<v>":
                self.take()
                return ("vload", b, ix)
            return ("load", b, ix)
        if tok == "(":
            a = self.expr()
            op = self.take()
            b = self.expr()
            self.take(")")
            if op in ("+", "-", "*", "/"):
                if self.peek() == "<v>":
                    self.take()
                    return ("vbin", op, a, b)
                return ("bin", op, a, b)
            if op in ("<", "<=", ">", ">=", "=="):
                return ("cmp", op, a, b)
            raise ValueError(f"unknown operator {op!r}")
        if tok in UNARY:
            self.take("(")
            a = self.expr()
            self.take(")")
            return ("un", tok, a)
        if tok in ("real", "int", "splat"):
            self.take("(")
            a = self.expr()
            self.take(")")
            return (tok, a)
        if tok == "select":
            self.take("(")
            c = self.expr()
            self.take(",")
            a = self.expr()
            self.take(",")
            b = self.expr()
            self.take(")")
            return ("select", c, a, b)
        m = re.fullmatch(r"([isnv])(\d+)", tok)
        if m:
            return ({"i": "iv", "s": "sv", "n": "si", "v": "vv"}[m.group(1)], int(m.group(2)))
        raise ValueError(f"unexpected token {tok!r}")


def parse_expr(s: str):
    p = _P(_tokens(s))
    e = p.expr()
    if p.peek() is not None:
        raise ValueError(f"trailing tokens in {s!r}")
    return e


# ----- statements -----------------------------------------------------------------

def _parse_body(lines, pos, depth):
    body = []
    pad = "  " * depth
    while pos < len(lines):
        line = lines[pos]
        if line == "  " * (depth - 1) + "}":
            return body, pos + 1
        if not line.startswith(pad):
            raise ValueError(f"bad indentation: {line!r}")
        s = line[len(pad):]
        m = re.fullmatch(r"for i(\d+) in 0\.\.(\d+) \{", s)
        if m:
            inner, pos = _parse_body(lines, pos + 1, depth + 1)
            body.append(("for", int(m.group(1)), int(m.group(2)), inner))
            continue
        if s.startswith("if ") and s.endswith(" {"):
            cond = parse_expr(s[3:-2])
            inner, pos = _parse_body(lines, pos + 1, depth + 1)
            body.append(("if", cond, inner))
            continue
        if s.startswith("%"):
            p = _P(_tokens(s))
            b = int(p.take()[1:])
            ix = p.index()
            op = p.take()
            if op not in ("=", "<v="):
                raise ValueError(f"cannot read store {s!r}")
            val = p.expr()
            if p.peek() is not None:
                raise ValueError(f"trailing tokens in {s!r}")
            body.append(("vstore" if op == "<v=" else "store", b, ix, val))
            pos += 1
            continue
        m = re.fullmatch(r"([isnv])(\d+) = (.*)", s)
        if m:
            kind = {"s": "set", "n": "seti", "i": "setl", "v": "vset"}[m.group(1)]
            body.append((kind, int(m.group(2)), parse_expr(m.group(3))))
            pos += 1
            continue
        raise ValueError(f"cannot read statement {s!r}")
    if depth == 1:
        raise ValueError("missing closing brace")
    return body, pos


def _count(body, k):
    """Largest variable numbers, for nloops/nreal/nint/nvec."""
    def ex(e):
        if not isinstance(e, tuple):
            return
        tag = e[0]
        if tag in ("iv", "sv", "si", "vv"):
            key = {"iv": "l", "sv": "r", "si": "i", "vv": "v"}[tag]
            k[key] = max(k[key], e[1] + 1)
            return
        for x in e[1:]:
            if isinstance(x, list):
                for y in x:
                    ex(y)
            else:
                ex(x)

    for s in body:
        tag = s[0]
        if tag == "for":
            k["l"] = max(k["l"], s[1] + 1)
            _count(s[3], k)
        elif tag == "if":
            ex(s[1])
            _count(s[2], k)
        elif tag in ("store", "vstore"):
            for x in s[2]:
                ex(x)
            ex(s[3])
        else:
            key = {"set": "r", "seti": "i", "setl": "l", "vset": "v"}[tag]
            k[key] = max(k[key], s[1] + 1)
            ex(s[2])


def parse_kernel(text: str) -> Kernel:
    lines = text.rstrip("\n").split("\n")
    head = lines[0]
    if not head.startswith("kernel ") or not head.endswith("{"):
        raise ValueError(f"not a kernel header: {head!r}")
    arrow = head.index(" -> %")
    open_ = head.rfind(" (", 0, arrow)
    name = head[len("kernel "):open_]
    ins = _split_specs(head[open_ + 2:arrow - 1])
    rest = head[arrow + len(" -> "):-1].rstrip()
    m = re.fullmatch(r"%(\d+) : (\S+?\[.*?\])( arith .*)?", rest)
    if not m or int(m.group(1)) != len(ins):
        raise ValueError(f"bad output spec {rest!r}")
    out = _parse_spec(m.group(2))
    arith = m.group(3).strip() if m.group(3) else None
    body, pos = _parse_body(lines, 1, 1)
    if pos != len(lines):
        raise ValueError("text after the kernel's closing brace")
    k = Kernel(name, ins, out, arith, body, text=text)
    cnt = {"l": 0, "r": 0, "i": 0, "v": 0}
    _count(body, cnt)
    k.nloops, k.nreal, k.nint, k.nvec = cnt["l"], cnt["r"], cnt["i"], cnt["v"]
    k.bufs = ins + [out]
    return k


def split_kernels(text: str) -> list:
    """Several kernels printed one after another (a snapshot)."""
    out, cur = [], []
    for line in text.split("\n"):
        if line.startswith("kernel "):
            cur = [line]
        elif cur:
            cur.append(line)
            if line == "}":
                out.append("\n".join(cur) + "\n")
                cur = []
    return out


# ----- printing back (the round trip that pins the reader) -------------------------

def _spec(b: Buf) -> str:
    axes = [f"{n}: {d}" if n is not None else str(d) for d, n in zip(b.dims, b.names)]
    return f"{b.ty}[{', '.join(axes)}]"


def show_expr(e) -> str:
    tag = e[0]
    if tag == "num":
        return e[1]
    if tag in ("load", "vload"):
        s = f"%{e[1]}[{', '.join(show_expr(x) for x in e[2])}]"
        return s + "<v>" if tag == "vload" else s
    if tag in ("iv", "sv", "si", "vv"):
        return {"iv": "i", "sv": "s", "si": "n", "vv": "v"}[tag] + str(e[1])
    if tag in ("bin", "vbin"):
        s = f"({show_expr(e[2])} {e[1]} {show_expr(e[3])})"
        return s + "<v>" if tag == "vbin" else s
    if tag == "cmp":
        return f"({show_expr(e[2])} {e[1]} {show_expr(e[3])})"
    if tag == "un":
        return f"{e[1]}({show_expr(e[2])})"
    if tag in ("real", "int", "splat"):
        return f"{tag}({show_expr(e[1])})"
    if tag == "select":
        return f"select({show_expr(e[1])}, {show_expr(e[2])}, {show_expr(e[3])})"
    raise ValueError(tag)


def _show_body(body, depth, out):
    pad = "  " * depth
    for s in body:
        tag = s[0]
        if tag == "for":
            out.append(f"{pad}for i{s[1]} in 0..{s[2]} {{")
            _show_body(s[3], depth + 1, out)
            out.append(pad + "}")
        elif tag == "if":
            out.append(f"{pad}if {show_expr(s[1])} {{")
            _show_body(s[2], depth + 1, out)
            out.append(pad + "}")
        elif tag in ("store", "vstore"):
            op = "<v=" if tag == "vstore" else "="
            out.append(f"{pad}%{s[1]}[{', '.join(show_expr(x) for x in s[2])}] {op} {show_expr(s[3])}")
        else:
            v = {"set": "s", "seti": "n", "setl": "i", "vset": "v"}[tag]
            out.append(f"{pad}{v}{s[1]} = {show_expr(s[2])}")


def show_kernel(k: Kernel) -> str:
    ins = ", ".join(f"%{i} : {_spec(b)}" for i, b in enumerate(k.inputs))
    arith = f" {k.arith}" if k.arith else ""
    out = [f"kernel {k.name} ({ins}) -> %{len(k.inputs)} : {_spec(k.output)}{arith} {{"]
    _show_body(k.body, 1, out)
    out.append("}")
    return "\n".join(out) + "\n"
