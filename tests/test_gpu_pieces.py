"""A KernelFn call split into pieces gives the whole call's bytes.

The native backend divides the iterations [0, n) of a nest's split loop
among its workers, each calling the kernel on [lo, hi), and its tests hold
that the result does not change by a bit (crates/presk-cranelift/src/
lib.rs:1656-1691, crates/presk-cranelift/tests/native.rs:331).  Here every
kernel class -- MFMA contractions (row, batch and split-K ranges; e8m15's
widen-multiply-narrow form too), the row
class, the column and scatter classes (whose nests have no split loop), and
the generic printer -- runs whole and then in 1, 2, 3 and 7 pieces into an
output poisoned with 0xff; the bytes must be equal."""
import numpy as np
import pytest

from presk_amd import hip
from presk_amd import lower as L
from tests import zoo

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand


def cases():
    out = []
    for dt in ("f32", "bf16", "f16"):
        x = O(A(("batch", 6), ("seq", 40), 96))
        w = O(A(96, 136))
        d = L.dot([x, w], dt)
        out.append((f"dot-{dt}", d, hip.FAST, "gemm"))
        out.append((f"dot+add-{dt}", L.dot([x, w, O(A(136))], dt, epilogue=(True, d.out_axes)), hip.FAST, "gemm"))
        out.append((f"dot_vjp_l-{dt}", L.dot_vjp_l([O(A(("batch", 5), ("seq", 130), 200)), O(A(72, 200))], dt), hip.FAST, "gemm"))
        # K = 4 x 600 over one 96 x 80 tile: split K, the range over I's rows
        out.append((f"dot_vjp_r-split-{dt}", L.dot_vjp_r([O(A(("batch", 4), ("seq", 600), 96)),
                                                          O(A(("batch", 4), ("seq", 600), 80))], dt), hip.FAST, "gemm"))
        q = O(A(("batch", 5), ("heads", 3), ("seq", 40), ("hd", 64)))
        kk = O(A(("batch", 5), ("heads", 3), ("seq2", 40), ("hd", 64)))
        out.append((f"ein_qk-{dt}", L.ein([q, kk], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]],
                                          ["batch", "heads", "seq", "seq2"], dt), hip.FAST, "gemm"))
        s = O(A(("batch", 5), ("heads", 3), ("seq", 40), ("seq2", 40)))
        mask = O(A(("seq", 40), ("seq2", 40)), "idx")
        out.append((f"masked_softmax-{dt}", L.masked_softmax("seq2", [s, mask], dt), hip.EXACT, "rows"))
        out.append((f"softmax2-{dt}", L.softmax_two_pass("seq2", [s], dt), hip.EXACT, "rows"))
        # long rows: the streamed kernel and the mask as bits (a workspace)
        sl = O(A(("batch", 3), ("heads", 2), ("seq", 300), ("seq2", 300)))
        ml = O(A(("seq", 300), ("seq2", 300)), "idx")
        out.append((f"masked_softmax_long-{dt}", L.masked_softmax("seq2", [sl, ml], dt), hip.EXACT, "rows"))
        logits = O(A(("batch", 7), ("seq", 60), ("vocab", 65)))
        ids = O(A(("batch", 7), ("seq", 60)), "idx")
        rows = O(A(("batch", 7), ("seq", 60)))
        out.append((f"mean-{dt}", L.reduce_axis("mean", "vocab", [logits], dt), hip.EXACT, "rows"))
        out.append((f"cross_entropy-{dt}", L.cross_entropy([logits, ids], dt), hip.EXACT, "rows"))
        out.append((f"cross_entropy_vjp-{dt}", L.cross_entropy_vjp([logits, ids, rows], dt), hip.EXACT, "rows"))
        # FAST's row nests (one wave a row, the lane-tree order)
        out.append((f"masked_softmax_fast-{dt}", L.masked_softmax("seq2", [s, mask], dt), hip.FAST, "rows"))
        out.append((f"mean_fast-{dt}", L.reduce_axis("mean", "vocab", [logits], dt), hip.FAST, "rows"))
        out.append((f"cross_entropy_vjp_fast-{dt}", L.cross_entropy_vjp([logits, ids, rows], dt), hip.FAST, "rows"))
        xs = O(A(("batch", 7), ("seq", 60), ("model", 96)))
        out.append((f"sum_to-{dt}", L.sum_to([xs, O(A(("model", 96)))], dt), hip.FAST, "colsum"))
        out.append((f"embed_vjp-{dt}", L.embed_vjp([O(A(("vocab", 65), ("model", 96))), ids, xs], dt), hip.EXACT, "scatter"))
        out.append((f"gelu-{dt}", L.unary("gelu", [xs], dt), hip.EXACT, "generic"))
        out.append((f"dot_exact-{dt}", d, hip.EXACT, "generic"))
    # e8m15 contractions (the f32 kernel on widened copies, then narrowed):
    # row, bias and split-K ranges
    x, w = O(A(("batch", 6), ("seq", 40), 96)), O(A(96, 136))
    d = L.dot([x, w], "e8m15")
    out.append(("dot-e8m15", d, hip.FAST, "gemm"))
    out.append(("dot+add-e8m15", L.dot([x, w, O(A(136))], "e8m15", epilogue=(True, d.out_axes)), hip.FAST, "gemm"))
    out.append(("dot_vjp_r-split-e8m15", L.dot_vjp_r([O(A(("batch", 4), ("seq", 600), 96)),
                                                       O(A(("batch", 4), ("seq", 600), 80))], "e8m15"), hip.FAST, "gemm"))
    # f32 products the planner puts on eight-wave tiles: the course step's
    # [16384 x 384] with a bias (256 x 96), the Linear module's [4096 x 1024]
    # (128 x 128), a batched ein over 16 entries (256 x 96)
    xc = O(A(("batch", 64), ("seq", 256), ("model", 384)))
    dc = L.dot([xc, O(A(384, 384))], "f32")
    out.append(("dot+add-f32-256x96", L.dot([xc, O(A(384, 384)), O(A(384))], "f32", epilogue=(True, dc.out_axes)),
                hip.FAST, "gemm"))
    out.append(("dot-f32-128x128-eight", L.dot([O(A(("batch", 4096), 1024)), O(A(1024, 1024))], "f32"), hip.FAST, "gemm"))
    out.append(("ein-batched-f32-256x96", L.ein([O(A(("b", 16), ("m", 1024), ("k", 384))), O(A(("b", 16), ("k", 384), ("n", 384)))],
                                                [["b", "m", "k"], ["b", "k", "n"]], ["b", "m", "n"], "f32"), hip.FAST, "gemm"))
    return out


def _run(c, ptrs, lo, hi):
    c.run(ptrs, lo, hi)


@pytest.mark.parametrize("case", cases(), ids=lambda c: c[0])
def test_pieces_equal_the_whole(case):
    name, low, mode, kind = case
    print(f"[pieces] {name}", flush=True)
    ex = hip.HipExec(0, mode=mode)
    c = ex.compiled(low.text, low.dtype, low.lanes)
    assert c.kind == kind, (c.kind, kind)
    ins = [hip.DeviceBuffer.of(a) for a in zoo.inputs(low, seed=3)]
    n_out = 1
    for a in low.out_axes:
        n_out *= a.len
    nbytes = max(n_out, 1) * hip.STORAGE_BYTES[low.dtype]
    out = hip.DeviceBuffer(nbytes)
    flag = hip.DeviceBuffer(4)
    flag.zero()
    ptrs = [b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else [])
    poison = np.full(nbytes, 0xFF, np.uint8)
    out.upload(poison)
    c.run(ptrs)
    hip.sync()
    whole = out.download(np.uint8)
    assert not np.array_equal(whole, poison)
    n = c.split_bound
    if kind in ("colsum", "scatter"):
        # these nests zero their output first: no split loop, whole calls only
        assert n == -1
        return
    assert n > 1, n
    for pieces in (1, 2, 3, 7):
        out.upload(poison)
        for t in range(pieces):
            lo, hi = n * t // pieces, n * (t + 1) // pieces
            c.run(ptrs, lo, hi)
        hip.sync()
        got = out.download(np.uint8)
        assert got.tobytes() == whole.tobytes(), f"{pieces} pieces of [0, {n})"
