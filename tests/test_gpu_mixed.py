"""A mixed realization (each site's storage type from a realization file, the
reference's schema): the course-GPT training step at TINY shapes with five
storage types, every kernel reading buffers of other types converted at its
edge.  EXACT mode: every launch's output equals the oracle's run of the same
program (its edge conversions the oracle's restatement of Buf::of), byte for
byte; the step as a graph equals the eager one."""
import numpy as np
import pytest

from presk_amd import configs, gpt, hip
from presk_amd.realize import Realization
from tests import cpu_program

pytestmark = pytest.mark.gpu

MIXED = Realization.of_json({
    "default": "bf16", "order": {"kind": "sequential"},
    "functions": {"LayerNorm.apply": "f32", "SelfAttention.apply": "f16", "MLP.apply": "bf16",
                  "Embedding.apply": "e8m15", "LayerNorm.apply.vjp": "f32", "MLP.apply.vjp": "f16"},
    "storage": {"MiniGPT.apply/logits": "f32", "MiniGPT.apply/ce": "f32", "MiniGPT.apply/loss": "f32",
                "SelfAttention.apply/probs": "f32"},
    "params": {"head": "f16", "blocks.ff.up.w": "bf16", "tok": "e8m15"}})


@pytest.mark.parametrize("train", [False, True])
def test_mixed_realization_exact(train):
    s = gpt.TINY
    p, b, names = gpt.build(s, "f32", train=train, mode=hip.EXACT, realize=MIXED)
    assert len({ln.low.dtype for ln in p.launches}) >= 4
    host = gpt.host_inputs(s)
    env = cpu_program.run(p, host)
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    assert any(st[0] == "convert" for st in p.steps)
    p.run()
    hip.sync()
    bad = [(ln.out, ln.low.name, ln.low.dtype) for ln in p.launches
           if p.bufs.download(ln.out).tobytes() != np.ascontiguousarray(env[ln.out]).tobytes()]
    assert not bad, f"{len(bad)} buffers differ, first: {bad[:5]}"
    assert bool(int(p._flag.download(np.uint32, 1)[0])) == env["__overflow__"]
    eager = {ln.out: p.bufs.download(ln.out).tobytes() for ln in p.launches}
    p.record(graph=True)
    for o in eager:
        p.bufs.dev[o].upload(np.full(p.bufs.dev[o].nbytes, 0x77, np.uint8))
    hip.sync()
    p.run()
    hip.sync()
    assert all(p.bufs.download(o).tobytes() == v for o, v in eager.items())
    p.release_batch()


@pytest.mark.parametrize("order", [{"kind": "interleaved", "partials": 4}, {"kind": "chunked", "size": 8}])
def test_declared_order_program_exact(order):
    """The course GPT's forward under a realization's reassociating order
    (every `dot` interleaved, or every contraction chunked): every buffer
    equals the oracle's run of the same nests."""
    s = gpt.TINY
    r = Realization.of_json({"default": "bf16", "order": order})
    print(f"[order] {order}", flush=True)
    p, b, names = gpt.build(s, "bf16", train=False, mode=hip.EXACT, realize=r)
    host = gpt.host_inputs(s)
    env = cpu_program.run(p, host)
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    bad = [ln.out for ln in p.launches if p.bufs.download(ln.out).tobytes() != np.ascontiguousarray(env[ln.out]).tobytes()]
    assert not bad, bad[:5]
