"""The FAST-mode column sum (`sum_to` onto trailing axes) in the executor's
own declared order, `rows-in-chunks(64)-f32`: chunks of 64 consecutive rows
each summed from zero in order, the chunk sums added in order from zero, in
f32 -- the shape of the reference's `ReductionOrder::Chunked { size: 64 }`
(crates/presk-kernel/src/lower.rs:427-464), which a realization applies to
contractions only.  The same order is written here as a PSK-Kernel nest and run by
the oracle; the device must give its bits exactly.  Also the row-nest class
at sizes beyond the zoo's, and the token scatter of `embed_vjp` over several
scan rounds, bit-exact against the oracle."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from tests import fmt, zoo

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand


def chunked_colsum_text(rows, cols, dtype, chunk=64):
    """out[c] = chunked sum over r of x[r, c] (x viewed [rows, cols])."""
    full, rem = divmod(rows, chunk)
    lines = [f"kernel colsum (%0 : {dtype}[{rows}, {cols}]) -> %1 : {dtype}[{cols}] {{",
             f"  for i0 in 0..{cols} {{", "    s0 = 0"]
    if full:
        lines += [f"    for i1 in 0..{full} {{", "      s1 = 0", f"      for i2 in 0..{chunk} {{",
                  f"        s1 = (s1 + %0[((i1 * {chunk}) + i2), i0])", "      }", "      s0 = (s0 + s1)", "    }"]
    if rem:
        lines += ["    s1 = 0", f"    for i2 in 0..{rem} {{", f"      s1 = (s1 + %0[(i2 + {full * chunk}), i0])", "    }",
                  "    s0 = (s0 + s1)"]
    lines += ["    %1[i0] = s0", "  }", "}"]
    return "\n".join(lines) + "\n"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(4, 300, 40), (64, 256, 384), (3, 5700, 70)])
def test_fast_sum_to_is_chunked_order(dt, shape):
    """one segment of chunk sums (19, 256 chunks) and two (268: a part
    chunk, a part column block, a second segment shorter than a batch)"""
    B, T, D = shape
    x = O(A(("batch", B), ("seq", T), ("model", D)))
    low = L.sum_to([x, O(A(("model", D)))], dt)
    ex = hip.HipExec(0, mode=hip.FAST)
    c = ex.compiled(low.text, dt, low.lanes)
    assert c.kind == "colsum", c.kind
    rng = np.random.default_rng(5)
    xs = fmt.encode(rng.standard_normal((B, T, D)).astype(np.float32), dt)
    want, _ = cexec.run(chunked_colsum_text(B * T, D, dt), dt, [xs, ], lanes=1)
    out = hip.DeviceBuffer(D * hip.STORAGE_BYTES[dt])
    ex.run(low.text, dt, [hip.DeviceBuffer.of(xs), hip.DeviceBuffer.of(np.zeros(D * hip.STORAGE_BYTES[dt], np.uint8))], out)
    assert out.download(want.dtype).tobytes() == want.tobytes()


def _big_rows(dt):
    B, H, T, V = 2, 3, 40, 65
    s = O(A(("batch", B), ("heads", H), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    logits = O(A(("batch", 5), ("seq", 60), ("vocab", V)))
    ids = O(A(("batch", 5), ("seq", 60)), "idx")
    rows = O(A(("batch", 5), ("seq", 60)))
    return [
        ("masked_softmax", L.masked_softmax("seq2", [s, mask], dt)),
        ("masked_softmax2", L.masked_softmax("seq2", [s, mask], dt, two_passes=True)),
        ("softmax", L.softmax("seq2", [s], dt)),
        ("mean", L.reduce_axis("mean", "vocab", [logits], dt)),
        ("cross_entropy", L.cross_entropy([logits, ids], dt)),
        ("cross_entropy_vjp", L.cross_entropy_vjp([logits, ids, rows], dt)),
        ("sum_to_rows", L.sum_to([logits, rows], dt)),
    ]


def _long_rows(dt):
    """rows longer than the four register-resident chunks (300 columns), and
    enough rows for sixteen rows a wave (65536)"""
    wide = O(A(("batch", 7), ("seq", 30), ("vocab", 300)))
    wide_rows = O(A(("batch", 7), ("seq", 30)))
    T = 256
    tall = O(A(("batch", 16), ("heads", 16), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    tall_wide = O(A(("batch", 1024), ("seq", 64), ("vocab", 300)))
    return [
        ("softmax", L.softmax("vocab", [wide], dt)),
        ("mean", L.reduce_axis("mean", "vocab", [wide], dt)),
        ("sum_to_rows", L.sum_to([wide, wide_rows], dt)),
        ("masked_softmax", L.masked_softmax("seq2", [tall, mask], dt)),
        ("softmax2", L.softmax_two_pass("vocab", [tall_wide], dt)),
    ]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_rows_class_exact_long_and_many(dt):
    ex = hip.HipExec(0, mode=hip.EXACT)
    from oracle import kernel_text as kt
    for name, low in _long_rows(dt):
        ins = zoo.inputs(low, seed=13, scale=2.0)
        if name == "masked_softmax":
            ins[1] = np.tril(np.ones((256, 256), np.int64)).ravel()
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes, threads=8)
        k = kt.parse_kernel(low.text)
        nbytes = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nbytes)
        out.upload(np.full(nbytes, 0xFF, np.uint8))
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", (name, c.kind)
        assert out.download(np.uint8, nbytes).tobytes() == want.view(np.uint8).tobytes(), name


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_rows_class_exact_at_size(dt):
    ex = hip.HipExec(0, mode=hip.EXACT)
    for name, low in _big_rows(dt):
        ins = zoo.inputs(low, seed=11, scale=3.0)
        if name == "masked_softmax" or name == "masked_softmax2":
            T = 40
            ins[1] = np.tril(np.ones((T, T), np.int64)).ravel()
        want, wf = cexec.run(low.text, dt, ins, lanes=low.lanes)
        from oracle import kernel_text as kt
        k = kt.parse_kernel(low.text)
        nbytes = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nbytes)
        out.upload(np.full(nbytes, 0xFF, np.uint8))
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", (name, c.kind)
        assert out.download(np.uint8, nbytes).tobytes() == want.view(np.uint8).tobytes(), name


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("ids", ["spread", "one_row"])
def test_scatter_class_exact_at_size(dt, ids):
    """embed_vjp over 4500 tokens (two scan rounds of 4096, the second
    partial) into a 7 x 300 table (a partial column block); with every token
    naming one row, a round's whole list is that row's (32 double batches of
    64 row loads, then a ragged 404)."""
    B, T, V, D = 3, 1500, 7, 300
    tok = O(A(("vocab", V), ("model", D)))
    idx = O(A(("batch", B), ("seq", T)), "idx")
    ct = O(A(("batch", B), ("seq", T), ("model", D)))
    low = L.embed_vjp([tok, idx, ct], dt)
    ins = zoo.inputs(low, seed=23)
    if ids == "one_row":
        ins[1] = np.full(B * T, 3, np.int64)
    want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
    ex = hip.HipExec(0, mode=hip.EXACT)
    nbytes = V * D * hip.STORAGE_BYTES[dt]
    out = hip.DeviceBuffer(nbytes)
    out.upload(np.full(nbytes, 0xFF, np.uint8))
    c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert c.kind == "scatter", c.kind
    assert out.download(np.uint8, nbytes).tobytes() == want.view(np.uint8).tobytes()


def _same_bits_nan_as_nan(got, want, dt):
    """bit-identical, except that any NaN matches any NaN (payloads of NaN
    arithmetic are not fixed by IEEE 754)"""
    g, w = fmt.decode(got, dt), fmt.decode(want, dt)
    gn, wn = np.isnan(g), np.isnan(w)
    assert (gn == wn).all(), np.argwhere(gn != wn)[:5]
    assert got.view(np.uint8).reshape(got.shape[0], -1)[~gn].tobytes() == want.view(np.uint8).reshape(want.shape[0], -1)[~wn].tobytes()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("T", [40, 256, 300, 320])
def test_rows_class_nan_and_empty_rows(dt, T):
    """the masked max's corner cases: a NaN first allowed element (the max is
    NaN), a NaN later allowed element and a NaN disallowed one (both passed
    over), -inf first, and a row the mask allows nowhere (all zeros); rows
    that stay in registers (40), short rows of whole 64-column chunks that
    are many enough to stream (256, 8192 rows), rows the long-row walk
    streams through the general row kernel (300, not whole 16-byte vectors)
    and through the streamed kernel (320)"""
    B, H = 2, (16 if T == 256 else 3)
    s = O(A(("batch", B), ("heads", H), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    ex = hip.HipExec(0, mode=hip.EXACT)
    from oracle import kernel_text as kt
    for low in (L.masked_softmax("seq2", [s, mask], dt), L.masked_softmax("seq2", [s, mask], dt, two_passes=True),
                L.softmax("seq2", [s], dt)):
        ins = zoo.inputs(low, seed=3)
        x = fmt.decode(ins[0], dt).reshape(B, H, T, T).copy()
        x[0, 0, 7, 0] = np.nan
        x[0, 1, 9, 4] = np.nan
        x[1, 2, 3, 20] = np.nan
        x[1, 0, 10, 0] = -np.inf
        x[1, 1, 12, 0] = np.nan if len(ins) == 1 else x[1, 1, 12, 0]
        ins[0] = fmt.encode(x.astype(np.float32), dt)
        if len(ins) == 2:
            m = np.tril(np.ones((T, T), np.int64))
            m[5, :] = 0
            ins[1] = m.ravel()
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
        k = kt.parse_kernel(low.text)
        nbytes = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nbytes)
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", c.kind
        got = out.download(want.dtype, want.size).reshape(want.shape)
        _same_bits_nan_as_nan(got, want, dt)


def chunked_total_text(n, dtype, mean, chunk=64, squares=False):
    """out = chunked sum of x[0..n) (chunks of 64 from zero, then the chunk sums
    in order from zero), divided by n for the mean: the declared order; with
    `squares` the terms are x * x (sum_squares)."""
    full, rem = divmod(n, chunk)
    lines = [f"kernel total (%0 : {dtype}[{n}]) -> %1 : {dtype}[] {{", "  s0 = 0"]
    term = (lambda i: f"(%0[{i}] * %0[{i}])") if squares else (lambda i: f"%0[{i}]")
    if full:
        lines += [f"  for i1 in 0..{full} {{", "    s1 = 0", f"    for i2 in 0..{chunk} {{",
                  f"      s1 = (s1 + {term(f'((i1 * {chunk}) + i2)')})", "    }", "    s0 = (s0 + s1)", "  }"]
    if rem:
        lines += ["  s1 = 0", f"  for i2 in 0..{rem} {{", f"    s1 = (s1 + {term(f'(i2 + {full * chunk})')})", "  }",
                  "  s0 = (s0 + s1)"]
    lines += [f"  %1[] = (s0 / {n})" if mean else "  %1[] = s0", "}"]
    return "\n".join(lines) + "\n"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("op", ["mean_all", "sum_all"])
@pytest.mark.parametrize("mode", [hip.FAST, hip.EXACT])
def test_totals(dt, op, mode):
    """sum_all / mean_all over 64 x 300 elements: FAST in the rows-in-chunks(64)
    order (colsum class), EXACT in index order through the long-row walk
    (rows class, one workgroup staging 4096 elements at a time)"""
    rows = O(A(("batch", 64), ("seq", 300)))
    low = L.reduce_all(op, [rows], dt)
    ex = hip.HipExec(0, mode=mode)
    ins = zoo.inputs(low, seed=7)
    c = ex.compiled(low.text, dt, low.lanes)
    if mode == hip.FAST:
        assert c.kind == "colsum", c.kind
        want, _ = cexec.run(chunked_total_text(64 * 300, dt, op == "mean_all"), dt, ins, lanes=1)
    else:
        assert c.kind == "rows", c.kind
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
    nb = hip.STORAGE_BYTES[dt]
    out = hip.DeviceBuffer(nb)
    ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert out.download(np.uint8, nb).tobytes() == want.view(np.uint8).tobytes()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_long_rows_exact(dt):
    """a few long rows (5 x 9000): mean and the stored running sum of
    `sum_to` onto leading axes, through the long-row walk, in index order"""
    x = O(A(("batch", 5), ("vocab", 9000)))
    r = O(A(("batch", 5)))
    ex = hip.HipExec(0, mode=hip.EXACT)
    from oracle import kernel_text as kt
    for low in (L.reduce_axis("mean", "vocab", [x], dt), L.sum_to([x, r], dt)):
        ins = zoo.inputs(low, seed=9)
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
        k = kt.parse_kernel(low.text)
        nb = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nb)
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", c.kind
        assert out.download(np.uint8, nb).tobytes() == want.view(np.uint8).tobytes(), low.name


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_long_row_walk_attention_shape(dt):
    """softmax over 2048-wide rows as an attention at Llama's context makes
    them (8192 rows, a causal mask over 2048 x 2048, the mask packed to bits):
    3 and 2 passes, masked and not, with NaNs, -inf and an empty mask row;
    and a row mean over 2048 x 4096 (RMSNorm's) -- every byte as the oracle's"""
    H, T = 4, 2048
    s = O(A(("batch", 1), ("heads", H), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    ex = hip.HipExec(0, mode=hip.EXACT)
    from oracle import kernel_text as kt
    cases = [L.masked_softmax("seq2", [s, mask], dt), L.masked_softmax("seq2", [s, mask], dt, two_passes=True),
             L.softmax("seq2", [s], dt), L.softmax_two_pass("seq2", [s], dt),
             L.reduce_axis("mean", "model", [O(A(("batch", 1), ("seq", 2048), ("model", 4096)))], dt)]
    for low in cases:
        print(f"[walk] {low.name} {dt}", flush=True)
        ins = zoo.inputs(low, seed=21, scale=4.0)
        if low.name.startswith("softmax"):
            x = fmt.decode(ins[0], dt).reshape(H, T, T).copy()
            x[0, 7, 0] = np.nan
            x[1, 9, 4] = np.nan
            x[2, 3, 1500] = np.nan
            x[3, 10, 0] = -np.inf
            x[0, 2047, 2047] = np.inf
            ins[0] = fmt.encode(x.astype(np.float32), dt)
        if len(ins) == 2:
            m = np.tril(np.ones((T, T), np.int64))
            m[5, :] = 0
            m[100, 50] = -3
            m[200, 300] = 7
            ins[1] = m.ravel()
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes, threads=8)
        k = kt.parse_kernel(low.text)
        nbytes = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nbytes)
        out.upload(np.full(nbytes, 0xFF, np.uint8))
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", c.kind
        got = out.download(want.dtype, want.size)
        _same_bits_nan_as_nan(got.reshape(-1), want.reshape(-1), dt)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("T", [64, 128, 192])
def test_short_rows_kept_in_registers(dt, T):
    """softmax rows of one, two and three 64-column chunks, at least 8 192 of
    them (the register-kept form): masked 3- and 2-pass and unmasked, a NaN,
    a row the mask allows nowhere, bit-exact against the oracle"""
    H = -(-8192 // T)
    s = O(A(("batch", 1), ("heads", H), ("seq", T), ("seq2", T)))
    mask = O(A(("seq", T), ("seq2", T)), "idx")
    ex = hip.HipExec(0, mode=hip.EXACT)
    from oracle import kernel_text as kt
    for low in (L.masked_softmax("seq2", [s, mask], dt), L.masked_softmax("seq2", [s, mask], dt, two_passes=True),
                L.softmax("seq2", [s], dt)):
        print(f"[short softmax] {dt} T={T} {low.name}", flush=True)
        ins = zoo.inputs(low, seed=23, scale=3.0)
        x = fmt.decode(ins[0], dt).reshape(H, T, T).copy()
        x[1, 3, 5] = np.nan
        ins[0] = fmt.encode(x.astype(np.float32), dt)
        if len(ins) == 2:
            m = np.tril(np.ones((T, T), np.int64))
            m[7, :] = 0
            ins[1] = m.ravel()
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes, threads=8)
        k = kt.parse_kernel(low.text)
        nbytes = k.output.numel * hip.STORAGE_BYTES[dt]
        out = hip.DeviceBuffer(nbytes)
        out.upload(np.full(nbytes, 0xFF, np.uint8))
        c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
        assert c.kind == "rows", c.kind
        got = out.download(want.dtype, want.size).reshape(want.shape)
        _same_bits_nan_as_nan(got, want, dt)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("mode", [hip.FAST, hip.EXACT])
@pytest.mark.parametrize("n", [1500, 590_000])
def test_sum_squares(dt, mode, n):
    """sum_squares (the optimizer's clipping, lower.rs:1693-1703): FAST in the
    rows-in-chunks(64) order with the terms x * x (colsum class: a part chunk, and
    9 219 chunks over two segments of the final chain), EXACT in index order;
    bit-exact against the oracle's run of the order as a nest"""
    x = O(A(("model", n)))
    low = L.sum_squares([x], dt)
    ex = hip.HipExec(0, mode=mode)
    ins = zoo.inputs(low, seed=31, scale=0.2)          # a total binary16 holds (590 000 x 0.04)
    c = ex.compiled(low.text, dt, low.lanes)
    if mode == hip.FAST:
        assert c.kind == "colsum", c.kind
        want, _ = cexec.run(chunked_total_text(n, dt, False, squares=True), dt, ins, lanes=1)
    else:
        want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
    nb = hip.STORAGE_BYTES[dt]
    out = hip.DeviceBuffer(nb)
    ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert out.download(np.uint8, nb).tobytes() == want.view(np.uint8).tobytes()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fast_sum_to_band_at_config4_size(dt):
    """The bias gradients' column sums at config 4's size ([64, 256, 384] ->
    [384]) against a float64 sum: two f32 orders of a sum of n terms differ
    by at most gamma_n sum|x| (n = 64 in a chunk + 256 chunk sums), plus one
    unit of the storage type for the stored total."""
    B, T, D = 64, 256, 384
    x = O(A(("batch", B), ("seq", T), ("model", D)))
    low = L.sum_to([x, O(A(("model", D)))], dt)
    ex = hip.HipExec(0, mode=hip.FAST)
    c = ex.compiled(low.text, dt, low.lanes)
    assert c.kind == "colsum" and c.order == "rows-in-chunks(64)-f32"
    rng = np.random.default_rng(11)
    xs = fmt.encode(rng.standard_normal((B, T, D)).astype(np.float32), dt)
    out = hip.DeviceBuffer(D * hip.STORAGE_BYTES[dt])
    ex.run(low.text, dt, [hip.DeviceBuffer.of(xs), hip.DeviceBuffer.of(np.zeros(D * hip.STORAGE_BYTES[dt], np.uint8))], out)
    got = fmt.decode(out.download(np.float32 if dt == "f32" else np.uint16), dt).astype(np.float64)
    xv = fmt.decode(xs, dt).astype(np.float64).reshape(B * T, D)
    exact = xv.sum(axis=0)
    n, u = 64 + B * T // 64, 2.0 ** -24
    ulp = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8}[dt]
    bound = n * u / (1 - n * u) * np.abs(xv).sum(axis=0) + ulp * np.abs(exact)
    assert np.all(np.abs(got - exact) <= bound)
