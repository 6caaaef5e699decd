"""Program.stack: buffers held one after another inside a stacked buffer
(the layers' slices of a `stack{L}` leaf), checked on the host."""
import pytest

from presk_amd import gpt, hip
from presk_amd.program import Buffers, Program


class _Parent:
    """A stand-in allocation: a base address and a size, nothing on a device."""
    def __init__(self, ptr, nbytes):
        self.ptr, self.nbytes = ptr, nbytes


def test_view_offsets_and_bounds():
    p = _Parent(4096, 64)
    v = hip.DeviceView(p, 16, 48)
    assert v.ptr == 4096 + 16 and v.nbytes == 48
    v.free()                                   # a view frees nothing
    assert p.ptr == 4096
    with pytest.raises(ValueError):
        hip.DeviceView(p, 32, 48)
    with pytest.raises(ValueError):
        hip.DeviceView(p, -4, 8)


def test_stack_records_each_member_at_its_slice():
    q = Program("t")
    q.stack("w", ["w0", "w1", "w2"], "f32", 10)
    assert q.bufs.views == {"w0": ("w", 0, "f32", 30), "w1": ("w", 10, "f32", 30), "w2": ("w", 20, "f32", 30)}
    with pytest.raises(ValueError):
        q.stack("w2x", ["w1"], "f32", 10)         # a buffer sits in one stack


def test_member_of_another_type_or_size_is_refused():
    b = Buffers()
    b.dev["w"], b.meta["w"] = _Parent(0, 120), ("f32", 30)
    b.views["w1"] = ("w", 10, "f32", 30)
    with pytest.raises(ValueError):
        b.alloc("w1", "bf16", 10)
    with pytest.raises(ValueError):
        b.views["w3"] = ("w", 25, "f32", 30)
        b.alloc("w3", "f32", 10)
    v = b.alloc("w1", "f32", 10)
    assert v.ptr == 40 and b.meta["w1"] == ("f32", 10)


def test_optimizer_leaves_stack_every_layer():
    s = gpt.TINY
    p, b, names = gpt.build(s, "f32", train=True, optimizer=True)
    leaves = gpt.opt_leaves(s)
    # a module's params, then its uses (crates/presk-types/src/elab/mod.rs:191-203)
    assert list(leaves)[:5] == ["tok", "pos", "head", "blocks.wq", "blocks.wq.b"]
    assert list(leaves)[-4:] == ["blocks.ln2.g", "blocks.ln2.b", "lnf.g", "lnf.b"]
    for n, (axes, members) in leaves.items():
        if members:
            assert axes[0].len == s.L and len(members) == s.L
            for l, m in enumerate(members):
                parent, first, ty, total = p.bufs.views[m]
                assert parent == n and ty == "f32" and first * s.L == l * total
                assert p.bufs.views[names["grads"][m]][0] == "d." + n
    assert set(names["adamw"]) == set(leaves)


def test_reference_checkpoint_layout_maps_onto_the_program():
    """`params GPT`'s leaves (a module's params, then its uses; Block's
    leaves stacked) name every stacked buffer and unstacked parameter once."""
    s = gpt.TINY
    layout, rename = gpt.params_layout(s)
    paths = layout.paths()
    assert paths[:4] == ["tok", "pos", "head", "blocks.attn.wq.w"] and paths[-2:] == ["lnf.γ", "lnf.β"]
    names = [rename.get(x, x) for x in paths]
    assert names == list(gpt.opt_leaves(s))
    assert [l.shape for l in layout.leaves()][3] == (s.L, s.D, s.D)
    p, b, _ = gpt.build(s, "f32", train=False)
    for n, (axes, members) in gpt.opt_leaves(s).items():
        if members:
            assert p.bufs.stacked(n) == ("f32", s.L * (p.bufs.views[members[0]][3] // s.L))
            assert [p.bufs.views[m][1] for m in members] == [l * p.bufs.views[members[0]][3] // s.L for l in range(s.L)]


def test_llama_checkpoint_layout_maps_onto_the_program():
    """`params Llama`: tok, head (its params), blocks, norm (its uses); every
    block leaf stacked over the layers in the program."""
    from presk_amd import llama
    s = llama.TINY
    layout, rename = llama.params_layout(s)
    paths = layout.paths()
    assert paths[:3] == ["tok", "head", "blocks.attn.wq"] and paths[-1] == "norm.γ"
    assert [rename.get(x, x) for x in paths] == list(llama.leaves(s))
    p, _, _ = llama.build(s, "bf16")
    for n, (axes, members) in llama.leaves(s).items():
        if members:
            assert p.bufs.stacked(n)[0] == "bf16" and [p.bufs.views[m][0] for m in members] == [n] * s.L
