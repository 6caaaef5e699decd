"""Fusion groups over a function body: `presk_core::fusion::plan`
(crates/presk-core/src/fusion.rs:138-230), restated over a body given as its
`let`s in order.

Backwards over the body, each elementwise `let` not yet claimed becomes the
root of a group that grows into its producers: a producer joins when it is
elementwise, of the root's type, not the body's result, not claimed, and
every one of its consumers is already in the group; a join that would make
the group's expression tree (a value read twice counted twice, `max`/`min`
reading each operand twice) exceed MAX_TREE nodes is undone.  Groups of one
member are not groups.  A group's steps are its members in body order, each
reading earlier steps or the group's inputs (first use order).

Values inside a group stay in the kernel's arithmetic type (f32 for bf16,
f16 and e8m15 storage, fusion.rs:1-9); everything else reaches memory in
its storage type.
"""
from __future__ import annotations

from dataclasses import dataclass, field

# PrimOp::elementwise (crates/presk-core/src/ir.rs:428-431), by this
# package's operator names (`pow2` is Pow(2), `pow1` Pow(1))
ELEMENTWISE = {"add", "sub", "mul", "div", "neg", "exp", "log", "tanh", "sqrt", "gelu", "relu", "abs", "sigmoid", "sin",
               "cos", "max", "min", "gelu_deriv", "heaviside", "sign", "pow1", "pow2"}
MAX_TREE = 64


@dataclass
class Let:
    var: str
    op: str                 # an elementwise op, or anything else (a literal, `real`, a call, a reduction)
    args: list
    ty: str                 # the result type: a group's members share it


@dataclass
class Group:
    root: str
    members: list
    inputs: list
    steps: list = field(default_factory=list)   # (op, [("in", i) | ("step", k)])
    ty: str = ""


def _tree_size(members: set, by_var: dict, root: str) -> int:
    budget = [MAX_TREE + 1]

    def go(v):
        if budget[0] == 0:
            return
        budget[0] -= 1
        if v not in members:
            return
        lt = by_var.get(v)
        if lt is None or lt.op not in ELEMENTWISE:
            return
        reads = 2 if lt.op in ("max", "min") else 1
        for a in lt.args:
            for _ in range(reads):
                go(a)
    go(root)
    return MAX_TREE + 1 - budget[0]


def plan(lets: list, result: str) -> dict:
    """{root: Group} of a body (its `let`s in order, `result` its value)."""
    by_var = {lt.var: lt for lt in lets}
    consumers: dict = {}
    for lt in lets:
        for a in lt.args:
            consumers.setdefault(a, []).append(lt.var)
    claimed: set = set()
    groups: dict = {}
    for lt in reversed(lets):
        if lt.var in claimed or lt.op not in ELEMENTWISE:
            continue
        members = {lt.var}
        while True:
            grew = False
            cands = [a for m in list(members) for a in by_var[m].args]
            for a in cands:
                if a in members or a in claimed or a == result:
                    continue
                p = by_var.get(a)
                if p is None or p.op not in ELEMENTWISE or p.ty != lt.ty:
                    continue
                if not all(c in members for c in consumers.get(a, [])):
                    continue
                members.add(a)
                if _tree_size(members, by_var, lt.var) > MAX_TREE:
                    members.discard(a)
                    continue
                grew = True
            if not grew:
                break
        if len(members) < 2:
            continue
        ordered = [m.var for m in lets if m.var in members]
        index = {v: i for i, v in enumerate(ordered)}
        inputs, steps = [], []
        for v in ordered:
            src = []
            for a in by_var[v].args:
                if a in index:
                    src.append(("step", index[a]))
                else:
                    if a not in inputs:
                        inputs.append(a)
                    src.append(("in", inputs.index(a)))
            steps.append((by_var[v].op, src))
        claimed.update(ordered)
        groups[lt.var] = Group(lt.var, ordered, inputs, steps, lt.ty)
    return groups
