"""A recorded launch sequence replayed as one HIP graph gives the eager
sequence's bits: the course-GPT training step (a reduced shape, FAST and
EXACT) eagerly, then recorded and replayed three times with eager device
work and host synchronisation between replays; every buffer of every replay
must equal the eager run's byte for byte.  With branches, the launches that
share no bytes lie on parallel branches of the graph."""
import numpy as np
import pytest

from presk_amd import configs, gpt, hip

pytestmark = pytest.mark.gpu

SMALL = gpt.GptShape(V=65, D=128, H=2, L=2, B=4, T=64)


BRANCHES_OFF = ("parallel graph branches are switched off: the branched capture of this test (f32, FAST, "
                "4 branches) ended in a host segmentation fault inside presk_hip_batch_graph_branches, cause not found")


@pytest.mark.parametrize("branches", [1, pytest.param(4, marks=pytest.mark.skip(reason=BRANCHES_OFF))])
@pytest.mark.parametrize("mode", [hip.FAST, hip.EXACT])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_graph_replays_match_eager(dt, mode, branches):
    s = SMALL
    p, b, names = gpt.build(s, dt, train=True, mode=mode)
    host = gpt.host_inputs(s)
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    outs = [ln.out for ln in p.launches]
    eager = {o: p.bufs.download(o).tobytes() for o in outs}
    p.record(graph=True, branches=branches)
    for rep in range(3):
        # scribble over every output so a replay that skips a launch shows
        for o in outs:
            p.bufs.dev[o].upload(np.full(p.bufs.dev[o].nbytes, 0xA5 + rep, np.uint8))
        hip.sync()
        p.run()
        hip.sync()
        bad = [o for o in outs if p.bufs.download(o).tobytes() != eager[o]]
        assert not bad, f"replay {rep}: {len(bad)} buffers differ, first {bad[:4]}"
        # eager work between replays: one launch of the sequence, alone
        ln = p.launches[len(p.launches) // 2]
        c = ln.compiled
        hip.check(hip.lib().presk_hip_run(c.handle, ln.table, 0, max(c.split_bound, 0), None))
        hip.sync()
    p.check_overflow()
    p.release_batch()


@pytest.mark.skip(reason=BRANCHES_OFF)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_llama_branched_graph_matches_eager(dt):
    """The Llama decoder forward (views, slices, concat, grouped-query ein),
    its launches on four branches: every buffer of two replays equals the
    eager run's."""
    from presk_amd import llama
    s = llama.LlamaShape(V=256, D=128, H=4, G=2, FF=192, L=2, B=2, T=64)
    print(f"[graph] llama {dt} branches 4", flush=True)
    p, b, names = llama.build(s, dt, mode=hip.FAST)
    p.compile()
    configs.load_inputs(p, llama.host_inputs(s))
    p.prepare()
    p.run()
    hip.sync()
    p.check_overflow()
    outs = [ln.out for ln in p.launches]
    eager = {o: p.bufs.download(o).tobytes() for o in outs}
    p.record(graph=True, branches=4)
    for rep in range(2):
        for o in outs:
            p.bufs.dev[o].upload(np.full(p.bufs.dev[o].nbytes, 0x5A + rep, np.uint8))
        hip.sync()
        p.run()
        hip.sync()
        bad = [o for o in outs if p.bufs.download(o).tobytes() != eager[o]]
        assert not bad, f"replay {rep}: {len(bad)} buffers differ, first {bad[:4]}"
    p.check_overflow()
    p.release_batch()
