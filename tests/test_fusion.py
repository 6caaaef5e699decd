"""The fusion planner (presk_amd/fusion.py, crates/presk-core/src/fusion.rs:138)
against the properties the reference's own test checks over its corpus
(crates/presk-realize/tests/plan.rs:38-92: a group has two members or more,
its root is its last member, members share the group's type, a member's
value never escapes the group, a step reads only earlier steps and the
group's inputs) and against cases whose grouping the rules fix: a diamond
(a value read twice inside one group joins), a value read by two groups (it
stays out), the body's result (never interior), a type boundary, the tree
limit (64 nodes, a value read twice counted twice, max/min reading each
operand twice), and adamw's bodies as optim.rs emits them."""
from presk_amd import fusion as FU
from presk_amd import gpt
from presk_amd.fusion import Let


def check_invariants(lets, result, groups):
    by = {l.var: l for l in lets}
    seen = set()
    for root, g in groups.items():
        assert len(g.members) >= 2 and g.members[-1] == root
        for m in g.members:
            assert m not in seen
            seen.add(m)
            assert by[m].ty == g.ty
            if m != root:
                assert m != result
                for l in lets:
                    if m in l.args:
                        assert l.var in g.members, (m, l.var)
        for i, (_, srcs) in enumerate(g.steps):
            for kind, k in srcs:
                assert (k < i) if kind == "step" else (k < len(g.inputs))
        assert len(g.steps) == len(g.members)


def test_diamond_and_shared_values():
    lets = [Let("a", "exp", ["x"], "t"), Let("b", "mul", ["a", "a"], "t"), Let("c", "add", ["b", "a"], "t"),
            Let("d", "neg", ["y"], "t"), Let("e", "mul", ["d", "x"], "t"), Let("f", "add", ["d", "y"], "t"),
            Let("r", "add", ["c", "e"], "t"), Let("out", "tuple", ["r", "f"], "u")]
    g = FU.plan(lets, "out")
    check_invariants(lets, "out", g)
    assert g["r"].members == ["a", "b", "c", "e", "r"]      # a is read by b twice and by c: all inside
    assert "d" not in g["r"].members and g["r"].inputs == ["x", "d"]
    assert "f" not in g                                       # f = d + y alone; d read by e and f
    assert [s[0] for s in g["r"].steps] == ["exp", "mul", "add", "mul", "add"]


def test_result_type_and_reduction_boundaries():
    lets = [Let("a", "exp", ["x"], "t"), Let("s", "sum", ["a"], "u"), Let("b", "neg", ["a"], "t"),
            Let("c", "log", ["s"], "u"), Let("d", "mul", ["b", "c"], "t")]
    g = FU.plan(lets, "b")
    check_invariants(lets, "b", g)
    assert list(g) == []          # b is the result; a is read by a reduction; c and d differ in type


def test_tree_limit():
    lets = [Let("v0", "exp", ["x"], "t")] + [Let(f"v{i}", "add", [f"v{i - 1}", "x"], "t") for i in range(1, 40)]
    g = FU.plan(lets, "v39")
    check_invariants(lets, "v39", g)
    sizes = [FU._tree_size(set(gr.members), {l.var: l for l in lets}, r) for r, gr in g.items()]
    assert all(s <= FU.MAX_TREE for s in sizes) and len(g) == 2       # 79 nodes do not fit one tree
    lets = [Let("a", "exp", ["x"], "t")] + [Let(f"m{i}", "max", [f"m{i - 1}" if i else "a", "y"], "t") for i in range(6)]
    g = FU.plan(lets, "z")
    # max reads each operand twice: the tree doubles a level, so 6 levels pass 64
    assert all(FU._tree_size(set(gr.members), {l.var: l for l in lets}, r) <= FU.MAX_TREE for r, gr in g.items())
    assert len(g) >= 2


def test_adamw_groups():
    lets, res = gpt._step_lets()
    g = FU.plan(lets, res)
    check_invariants(lets, res, g)
    assert g["theta2"].members == ["mhat", "vhat", "sq", "den", "upd", "decay", "dir", "scaled", "theta2"]
    assert g["m2"].members == ["ma", "mc", "m2"] and g["v2"].members == ["va", "gg", "vc", "v2"]
    assert g["factor"].members == ["norm", "denom", "coef", "fd", "fr", "factor"]
    assert "gc" not in g and "omb1" not in g          # the clipped gradient feeds two groups; 1 - b1 alone
    lets, res = gpt._lr_lets()
    g = FU.plan(lets, res)
    check_invariants(lets, res, g)
    assert list(g) == ["lr"] and len(g["lr"].members) == 20      # the schedule is one nest
