"""The MFMA contraction class (FAST mode) against the oracle's sequential
sums, within the band the reassociation allows.

The executor's order is declared (its kernel info names it): MFMA tiles with
f32 accumulation, k-blocks in increasing order, split-K partials added in
split order.  Two f32 orders of one sum of K terms differ by at most
2*gamma_K*sum|x_k w_k| (gamma_K = K u / (1 - K u), u = 2^-24); a narrow
storage type adds at most one unit in its last place per store, of the sum
(at most sum|x_k w_k|) and of the result.  Every element must be within that bound, and the bulk far inside it
(median error below 1/64 of the bound), so a misplaced operand or a lost
k-block cannot pass."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand

ULP = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10, "e8m15": 2.0 ** -15}


def cases():
    out = []
    for dt in ("f32", "bf16", "f16"):
        x = O(A(("batch", 3), ("seq", 200), 96))
        w = O(A(96, 136))
        d = L.dot([x, w], dt)
        out.append((f"dot-{dt}", d, None))
        out.append((f"dot+add-{dt}", L.dot([x, w, O(A(136))], dt, epilogue=(True, d.out_axes)), None))
        out.append((f"dot_vjp_l-{dt}", L.dot_vjp_l([O(A(("batch", 2), ("seq", 130), 200)), O(A(72, 200))], dt), None))
        out.append((f"dot_vjp_r-split-{dt}", L.dot_vjp_r([O(A(("batch", 4), ("seq", 600), 96)), O(A(("batch", 4), ("seq", 600), 80))], dt), None))
        # whole k-blocks (f32 tiles then load straight into LDS): both operands
        # k-contiguous with rows past a tile, and an m-contiguous operand of
        # 100 rows whose last vectors are clamped
        out.append((f"dot_vjp_l-k192-{dt}", L.dot_vjp_l([O(A(("batch", 2), ("seq", 130), 192)), O(A(72, 192))], dt), None))
        out.append((f"dot_vjp_r-m100-{dt}", L.dot_vjp_r([O(A(("batch", 4), ("seq", 600), 100)), O(A(("batch", 4), ("seq", 600), 76))], dt), None))
        q = O(A(("batch", 2), ("heads", 3), ("seq", 40), ("hd", 64)))
        kk = O(A(("batch", 2), ("heads", 3), ("seq2", 40), ("hd", 64)))
        s = O(A(("batch", 2), ("heads", 3), ("seq", 40), ("seq2", 40)))
        out.append((f"ein_qk-{dt}", L.ein([q, kk], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]], ["batch", "heads", "seq", "seq2"], dt), None))
        out.append((f"ein_av-{dt}", L.ein([s, kk], [["batch", "heads", "seq", "seq2"], ["batch", "heads", "seq2", "hd"]], ["batch", "heads", "seq", "hd"], dt), None))
        # 128 x 96 tiles (N = 384 over 16384 rows fills the CUs in 4 column
        # tiles): NN and NT; the 128 x 64 tiles are the ein_av cases above
        xb = O(A(("batch", 8), ("seq", 2048), 200))
        out.append((f"dot+add-bn96-{dt}", L.dot([xb, O(A(200, 384)), O(A(384))], dt, epilogue=(True, A(("batch", 8), ("seq", 2048), 384))), None))
        out.append((f"dot_vjp_l-bn96-{dt}", L.dot_vjp_l([xb, O(A(384, 200))], dt), None))
        # the Llama attention's `ein`s (grouped-query: 2 groups of 3 heads):
        # projections that broadcast an operand over batch axes, scores and
        # values whose rows are not the output's second-last axis, and an
        # output projection summed over three axes read as one K
        xq = O(A(("batch", 2), ("seq", 100), ("model", 64)))
        wq3 = O(A(("model", 64), ("groups", 2), ("per", 3), ("hd", 32)))
        out.append((f"ein_qproj-{dt}", L.ein([xq, wq3], [["batch", "seq", "model"], ["model", "groups", "per", "hd"]],
                                             ["batch", "groups", "per", "seq", "hd"], dt), None))
        qg = O(A(("batch", 2), ("groups", 2), ("per", 3), ("seq", 100), ("hd", 32)))
        kg = O(A(("batch", 2), ("groups", 2), ("seq", 100), 32))
        out.append((f"ein_gqa_scores-{dt}", L.ein([qg, kg], [["batch", "groups", "per", "seq", "hd"], ["batch", "groups", "seq2", "hd"]],
                                                  ["batch", "groups", "per", "seq", "seq2"], dt), None))
        ag = O(A(("batch", 2), ("groups", 2), ("per", 3), ("seq", 100), ("seq2", 100)))
        vg = O(A(("batch", 2), ("seq", 100), ("groups", 2), ("hd", 32)))
        out.append((f"ein_gqa_values-{dt}", L.ein([ag, vg], [["batch", "groups", "per", "seq", "seq2"], ["batch", "seq2", "groups", "hd"]],
                                                  ["batch", "seq", "groups", "per", "hd"], dt), None))
        og = O(A(("batch", 2), ("seq", 100), ("groups", 2), ("per", 3), ("hd", 32)))
        w2 = O(A(("groups", 2), ("per", 3), ("hd", 32), ("model", 72)))
        out.append((f"ein_oproj-{dt}", L.ein([og, w2], [["batch", "seq", "groups", "per", "hd"], ["groups", "per", "hd", "model"]],
                                             ["batch", "seq", "model"], dt), None))
    # 16-bit storage, whole k-blocks, aligned vectors below K 3072: the
    # 128-row tiles in each operand layout (the 256-row tiles at K >= 3072
    # are test_d16_tiles_within_band's)
    for dt in ("bf16", "f16"):
        out.append((f"d16-nn-{dt}", L.dot([O(A(("batch", 3), ("seq", 300), 320)), O(A(320, 200))], dt), None))
        out.append((f"d16-nt-{dt}", L.dot_vjp_l([O(A(("batch", 2), ("seq", 130), 128)), O(A(264, 128))], dt), None))
        out.append((f"d16-tn-{dt}", L.dot_vjp_r([O(A(("batch", 4), ("seq", 96), 104)), O(A(("batch", 4), ("seq", 96), 136))], dt), None))
        out.append((f"d16-tt-{dt}", L.ein([O(A(("k", 64), ("m", 264))), O(A(("n", 72), ("k", 64)))], [["k", "m"], ["n", "k"]],
                                          ["m", "n"], dt), None))
        out.append((f"d16-bias-{dt}", L.dot([O(A(("batch", 520), 384)), O(A(384, 256)), O(A(256))], dt,
                                            epilogue=(True, A(("batch", 520), 256))), None))
    # e8m15: the codes widened exactly to f32, the f32 kernel, the sums
    # narrowed (with the bias added after the first rounding)
    x, w = O(A(("batch", 3), ("seq", 200), 96)), O(A(96, 136))
    d = L.dot([x, w], "e8m15")
    out.append(("dot-e8m15", d, None))
    out.append(("dot+add-e8m15", L.dot([x, w, O(A(136))], "e8m15", epilogue=(True, d.out_axes)), None))
    out.append(("dot_vjp_l-e8m15", L.dot_vjp_l([O(A(("batch", 2), ("seq", 130), 200)), O(A(72, 200))], "e8m15"), None))
    out.append(("dot_vjp_r-split-e8m15", L.dot_vjp_r([O(A(("batch", 4), ("seq", 600), 96)),
                                                       O(A(("batch", 4), ("seq", 600), 80))], "e8m15"), None))
    q = O(A(("batch", 2), ("heads", 3), ("seq", 40), ("hd", 64)))
    kk = O(A(("batch", 2), ("heads", 3), ("seq2", 40), ("hd", 64)))
    out.append(("ein_qk-e8m15", L.ein([q, kk], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]],
                                      ["batch", "heads", "seq", "seq2"], "e8m15"), None))
    # a K that is not a multiple of the k-block, M and N below one tile
    out.append(("dot-odd-bf16", L.dot([O(A(("batch", 5), 77)), O(A(77, 24))], "bf16"), None))
    return out


def abs_products(low, vals):
    """sum_k |x_k w_k| per output element, in f64, via the oracle on |x|, |w| in f64."""
    text = low.text.replace(f": {low.dtype}[", ": f64[")
    absv = [np.abs(v.astype(np.float64)) for v in vals]
    if low.name.endswith("+add"):
        absv[2] = np.zeros_like(absv[2])
    out, _ = cexec.run(text, "f64", [a.ravel() for a in absv], lanes=low.lanes)
    return out


@pytest.fixture(scope="module")
def ex():
    return hip.HipExec(0, mode=hip.FAST)


@pytest.mark.parametrize("case", cases(), ids=lambda c: c[0])
def test_fast_contraction_within_band(ex, case):
    name, low, _ = case
    print(f"[gemm] {name}", flush=True)
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(3)
    vals = [fmt.roundtrip(rng.standard_normal(b.dims).astype(np.float32), low.dtype) for b in k.inputs]
    ins = [fmt.encode(v, low.dtype) for v in vals]
    want, _ = cexec.run(low.text, low.dtype, ins, lanes=low.lanes)
    nbytes = k.output.numel * hip.STORAGE_BYTES[low.dtype]
    out = hip.DeviceBuffer(nbytes)
    out.upload(np.full(nbytes, 0xFF, np.uint8))
    c = ex.run(low.text, low.dtype, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert c.kind == "gemm", c.kind
    got = fmt.decode(out.download(want.dtype), low.dtype).astype(np.float64)
    ref = fmt.decode(want, low.dtype).astype(np.float64)
    K = c.flops / (2 * k.output.numel)
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    S = abs_products(low, vals)
    # a narrow store of the sum can differ by one unit of |sum| <= S, which a
    # bias that cancels carries into a smaller result
    bound = 2 * gamma * S + ULP[low.dtype] * (S + 2 * np.maximum(np.abs(ref), np.abs(got))) + 1e-30
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got)), f"{name}: unwritten or non-finite outputs"
    assert np.all(err <= bound), f"{name} [{c.order}]: {np.count_nonzero(err > bound)} elements outside the band"
    assert np.median(err / bound) < 1 / 64, f"{name}: median error {np.median(err / bound):.3g} of the band"


# K >= 3072, whole k-blocks, aligned vectors, no k-split: the eight-wave
# 256-row tiles of 32x32x16 MFMAs loaded straight into LDS -- 256 x 128
# (three k-blocks deep) and, where they make three rounds of the CUs,
# 256 x 256 (two k-blocks deep, the sums staged in two halves) -- and, under
# PRESK_HIP_GEMM_TILE, the four-wave 128 x 128 tiles.  Each operand layout
# (k-contiguous or not), every remainder of the stage rounds, rows past a
# tile, the bias.  Every output must be written (the buffer is poisoned with
# NaNs) and 20 000 sampled elements must lie within gamma_K S plus the
# storage type's unit of the sum and the result of the f64 product of the
# same rounded operands.
D16 = {
    "nn": (lambda dt: L.dot([O(A(("batch", 1100), 3136)), O(A(3136, 4104))], dt), "ab", 256 * 128),
    "nt": (lambda dt: L.dot_vjp_l([O(A(("batch", 2056), 3200)), O(A(2048, 3200))], dt), "abT", 256 * 128),
    "tn": (lambda dt: L.dot_vjp_r([O(A(("batch", 3072), 2048)), O(A(("batch", 3072), 2056))], dt), "aTb", 256 * 128),
    "tt": (lambda dt: L.ein([O(A(("k", 3072), ("m", 2048))), O(A(("n", 2048), ("k", 3072)))], [["k", "m"], ["n", "k"]],
                            ["m", "n"], dt), "aTbT", 256 * 128),
    "bias": (lambda dt: L.dot([O(A(("batch", 2048), 3072)), O(A(3072, 2048)), O(A(2048))], dt,
                              epilogue=(True, A(("batch", 2048), 2048))), "ab", 256 * 128),
    "nn256": (lambda dt: L.dot([O(A(("batch", 2056), 3136)), O(A(3136, 24584))], dt), "ab", 256 * 256),
    "nt256": (lambda dt: L.dot_vjp_l([O(A(("batch", 24584), 3072)), O(A(2056, 3072))], dt), "abT", 256 * 256),
    "tn256": (lambda dt: L.dot_vjp_r([O(A(("batch", 3072), 2056)), O(A(("batch", 3072), 24584))], dt), "aTb", 256 * 256),
    "tt256": (lambda dt: L.ein([O(A(("k", 3136), ("m", 24584))), O(A(("n", 2056), ("k", 3136)))], [["k", "m"], ["n", "k"]],
                               ["m", "n"], dt), "aTbT", 256 * 256),
}


# the 256 x 256 tiles are the same code in f16 as in bf16: bf16 covers them at size
@pytest.mark.parametrize("layout,dt,tiles", [(lay, dt, None) for lay in D16 for dt in ("bf16", "f16")
                                             if dt == "bf16" or D16[lay][2] <= 256 * 128]
                         + [("nn", "bf16", "128x128"), ("tt", "bf16", "128x128"), ("tn", "f16", "128x128")])
def test_d16_tiles_within_band(ex, layout, dt, tiles, monkeypatch):
    from oracle import kernel_text as kt
    mk, form, tile = D16[layout]
    low = mk(dt)
    if tiles:
        monkeypatch.setenv("PRESK_HIP_GEMM_TILE", tiles)
    print(f"[gemm] d16 {layout} {dt} {tiles or ''}", flush=True)
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(5)
    vals = [fmt.roundtrip(rng.standard_normal(b.dims, dtype=np.float32), dt) for b in k.inputs]
    out = hip.DeviceBuffer(k.output.numel * 2)
    out.upload(np.full(k.output.numel * 2, 0xFF, np.uint8))
    c = ex.run(low.text, dt, [hip.DeviceBuffer.of(fmt.encode(v, dt)) for v in vals], out, lanes=low.lanes)
    assert c.kind == "gemm" and c.order == "mfma-k16", (c.kind, c.order)
    got = fmt.decode(out.download(np.uint16), dt).reshape(k.output.dims)
    assert np.all(np.isfinite(got)), "unwritten or non-finite outputs"
    a, b = vals[0].reshape(k.inputs[0].dims), vals[1].reshape(k.inputs[1].dims)
    a = a.T if form.startswith("aT") else a            # [M, K]
    b = b.T if form.endswith("bT") else b              # [K, N]
    Mo, No = got.shape
    ms, ns = rng.integers(0, Mo, 20000), rng.integers(0, No, 20000)
    exact, S = np.empty(len(ms)), np.empty(len(ms))
    for c0 in range(0, len(ms), 2000):
        ra, cb = a[ms[c0:c0 + 2000]].astype(np.float64), b[:, ns[c0:c0 + 2000]].T.astype(np.float64)
        exact[c0:c0 + 2000] = np.einsum("ik,ik->i", ra, cb)
        S[c0:c0 + 2000] = np.einsum("ik,ik->i", np.abs(ra), np.abs(cb))
    if layout == "bias":
        exact = fmt.roundtrip(exact.astype(np.float32), dt).astype(np.float64) + vals[2][ns].astype(np.float64)
    g = got[ms, ns].astype(np.float64)
    K = a.shape[1]
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    bound = gamma * S + ULP[dt] * (S + 2 * np.maximum(np.abs(exact), np.abs(g))) + 1e-30
    err = np.abs(g - exact)
    assert np.all(err <= bound), f"{np.count_nonzero(err > bound)} sampled elements outside the band"
    assert np.median(err / bound) < 1 / 16, f"median error {np.median(err / bound):.3g} of the band"


# The eight-wave 256-row tiles (two waves a SIMD) compute each output with
# the same 32x32x16 MFMAs over the same k-steps as the four-wave 128 x 128
# tiles, so the two must agree bit for bit -- in every operand layout, with
# rows and columns past the last tile, and with the bias.
EIGHT = {
    "nn": lambda dt: L.dot([O(A(("batch", 1040), 1024)), O(A(1024, 392))], dt),
    "nt": lambda dt: L.dot_vjp_l([O(A(("batch", 520), 768)), O(A(648, 768))], dt),
    "tn": lambda dt: L.dot_vjp_r([O(A(("batch", 1024), 264)), O(A(("batch", 1024), 520))], dt),
    "tt": lambda dt: L.ein([O(A(("k", 832), ("m", 776))), O(A(("n", 264), ("k", 832)))], [["k", "m"], ["n", "k"]],
                           ["m", "n"], dt),
    "bias": lambda dt: L.dot([O(A(("batch", 1288), 768)), O(A(768, 520)), O(A(520))], dt,
                             epilogue=(True, A(("batch", 1288), 520))),
    # a batched ein: each batch entry's tiles at its own offsets
    "batched": lambda dt: L.ein([O(A(("b", 3), ("m", 520), ("k", 384))), O(A(("b", 3), ("k", 384), ("n", 264)))],
                                [["b", "m", "k"], ["b", "k", "n"]], ["b", "m", "n"], dt),
}


@pytest.mark.parametrize("layout,dt,tiles", [(lay, "bf16", t) for lay in EIGHT for t in ("256x128", "256x256")]
                         + [("nn", "f16", "256x128"), ("tt", "f16", "256x256")])
def test_eight_wave_tiles_equal_the_128_row_tiles(layout, dt, tiles, monkeypatch):
    from oracle import kernel_text as kt
    low = EIGHT[layout](dt)
    print(f"[gemm] eight waves {layout} {dt} {tiles}", flush=True)
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(9)
    ins = [hip.DeviceBuffer.of(fmt.encode(fmt.roundtrip(rng.standard_normal(b.dims, dtype=np.float32), dt), dt))
           for b in k.inputs]
    outs = []
    # (the 128 x 128 tiles unsplit: a k-split adds its partials in another order)
    for t in (tiles, "128x128/1"):
        monkeypatch.setenv("PRESK_HIP_GEMM_TILE", t)
        c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
        assert c.kind == "gemm" and c.order == "mfma-k16", (c.kind, c.order)
        out = hip.DeviceBuffer(k.output.numel * 2)
        out.upload(np.full(k.output.numel * 2, 0xFF, np.uint8))
        flag = hip.DeviceBuffer(4)
        flag.zero()
        c.run([b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else []))
        hip.sync()
        outs.append(out.download(np.uint16))
    differ = np.count_nonzero(outs[0] != outs[1])
    assert differ == 0, f"{differ} of {outs[0].size} outputs differ from the 128 x 128 tiles'"


# The f32 eight-wave tiles (256 x 128 and 256 x 96, three 32-deep k-blocks
# straight into LDS, a 96-row B tile's last round of loads issued by half the
# waves) run the 16x16x4 MFMAs over the same k-steps as the four-wave 128-row
# tiles, so the two agree bit for bit -- in every operand layout, with rows
# and columns past the last tile, every remainder of the stage rounds, and
# with the bias.  Operands that the wide tiles cannot take (a row off 16
# bytes) run the 128-row tiles of the same columns, the same bits again.
@pytest.mark.parametrize("layout,tiles", [(lay, t) for lay in EIGHT for t in ("256x128", "256x96", "128x96w8/1")])
def test_f32_eight_wave_tiles_equal_the_128_row_tiles(layout, tiles, monkeypatch):
    from oracle import kernel_text as kt
    low = EIGHT[layout]("f32")
    print(f"[gemm] f32 eight waves {layout} {tiles}", flush=True)
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(11)
    ins = [hip.DeviceBuffer.of(rng.standard_normal(b.dims, dtype=np.float32)) for b in k.inputs]
    outs = []
    for t in (tiles, "128x128/1"):
        monkeypatch.setenv("PRESK_HIP_GEMM_TILE", t)
        c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
        assert c.kind == "gemm" and c.order == "mfma-f32-k4", (c.kind, c.order)
        out = hip.DeviceBuffer(k.output.numel * 4)
        out.upload(np.full(k.output.numel * 4, 0xFF, np.uint8))
        c.run([b.ptr for b in ins] + [out.ptr])
        hip.sync()
        outs.append(out.download(np.uint32))
    assert not np.any(outs[1] == 0xFFFFFFFF), "unwritten outputs"
    differ = np.count_nonzero(outs[0] != outs[1])
    assert differ == 0, f"{differ} of {outs[0].size} outputs differ from the 128 x 128 tiles'"


def test_f32_eight_wave_tiles_on_a_misaligned_operand(monkeypatch):
    # the A operand one element past a 16-byte boundary: the 256-row plan
    # falls back to 128-row tiles at launch, and the bits stay those of the
    # aligned run
    from oracle import kernel_text as kt
    low = EIGHT["nn"]("f32")
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(12)
    a = rng.standard_normal(k.inputs[0].numel, dtype=np.float32)
    b = rng.standard_normal(k.inputs[1].numel, dtype=np.float32)
    big = hip.DeviceBuffer(4 * (a.size + 4))
    big.upload(np.concatenate([np.zeros(1, np.float32), a, np.zeros(3, np.float32)]))
    a_al, b_d = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(b)
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "256x96")
    c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    outs = []
    for ptr in (a_al.ptr, big.ptr + 4):
        out = hip.DeviceBuffer(k.output.numel * 4)
        out.upload(np.full(k.output.numel * 4, 0xFF, np.uint8))
        c.run([ptr, b_d.ptr, out.ptr])
        hip.sync()
        outs.append(out.download(np.uint32))
    assert not np.any(outs[1] == 0xFFFFFFFF), "unwritten outputs"
    assert np.array_equal(outs[0], outs[1])


# The 128 x 128 tiles of eight waves (four k-blocks in flight, for split-K
# weight gradients), f32 and 16-bit, against the four-wave tiles at the same
# split: the same partial sums, added in the same order, so the same bits.
@pytest.mark.parametrize("layout,splits,dt", [("tn", 1, "f32"), ("tn", 5, "f32"), ("nn", 3, "f32"), ("nt", 1, "f32"),
                                              ("tt", 4, "f32"), ("bias", 2, "f32"), ("tn", 1, "bf16"),
                                              ("tn", 3, "bf16"), ("nn", 2, "bf16"), ("nt", 1, "f16"),
                                              ("tt", 2, "bf16"), ("bias", 2, "f16")])
def test_eight_wave_128_tiles_equal_the_four_wave_tiles(layout, splits, dt, monkeypatch):
    from oracle import kernel_text as kt
    low = EIGHT[layout](dt)
    print(f"[gemm] eight waves 128x128 {layout} {dt} split {splits}", flush=True)
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(13)
    vals = [rng.standard_normal(b.dims, dtype=np.float32) for b in k.inputs]
    ins = [hip.DeviceBuffer.of(v if dt == "f32" else fmt.encode(fmt.roundtrip(v, dt), dt)) for v in vals]
    esz, code = (4, np.uint32) if dt == "f32" else (2, np.uint16)
    outs = []
    for t in (f"128x128w8/{splits}", f"128x128/{splits}"):
        monkeypatch.setenv("PRESK_HIP_GEMM_TILE", t)
        c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
        want = ("mfma-f32-k4" if dt == "f32" else "mfma-k16") + (f"-split{splits}" if splits > 1 else "")
        assert c.kind == "gemm" and c.order == want, (c.kind, c.order)
        out = hip.DeviceBuffer(k.output.numel * esz)
        out.upload(np.full(k.output.numel * esz, 0xFF, np.uint8))
        flag = hip.DeviceBuffer(4)
        flag.zero()
        c.run([b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else []))
        hip.sync()
        outs.append(out.download(code))
    assert not np.any(outs[1] == code(-1 & (0xFFFFFFFF if dt == "f32" else 0xFFFF))), "unwritten outputs"
    differ = np.count_nonzero(outs[0] != outs[1])
    assert differ == 0, f"{differ} of {outs[0].size} outputs differ from the four-wave tiles'"


# Short K (one, two and three k-blocks: fewer than the stages in flight) and
# operands smaller than a tile on the eight-wave tiles, against the
# four-wave 128 x 128 tiles, bit for bit.
SHORT = [(100, 32, 72, "f32"), (300, 64, 200, "f32"), (520, 96, 136, "f32"), (40, 128, 392, "f32"),
         (100, 64, 72, "bf16"), (300, 128, 200, "bf16"), (520, 192, 136, "f16")]


# (256 x 96 and eight-wave 128 x 96 tiles are f32's only)
@pytest.mark.parametrize("m,k,n,dt,tiles", [(*s, t) for s in SHORT for t in ("256x128", "256x96", "128x128w8/1", "128x96w8/1")
                                            if s[3] == "f32" or t in ("256x128", "128x128w8/1")])
def test_eight_wave_tiles_short_k_and_small_operands(m, k, n, dt, tiles, monkeypatch):
    from oracle import kernel_text as kt
    low = L.dot([O(A(("batch", m), k)), O(A(k, n)), O(A(n))], dt, epilogue=(True, A(("batch", m), n)))
    print(f"[gemm] short {m}x{k}x{n} {dt} {tiles}", flush=True)
    kn = kt.parse_kernel(low.text)
    rng = np.random.default_rng(m + k + n)
    vals = [rng.standard_normal(b.dims, dtype=np.float32) for b in kn.inputs]
    ins = [hip.DeviceBuffer.of(v if dt == "f32" else fmt.encode(fmt.roundtrip(v, dt), dt)) for v in vals]
    esz, code = (4, np.uint32) if dt == "f32" else (2, np.uint16)
    outs = []
    for t in (tiles, "128x128/1"):
        monkeypatch.setenv("PRESK_HIP_GEMM_TILE", t)
        c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
        assert c.kind == "gemm" and "split" not in c.order, (c.kind, c.order)
        out = hip.DeviceBuffer(kn.output.numel * esz)
        out.upload(np.full(kn.output.numel * esz, 0xFF, np.uint8))
        flag = hip.DeviceBuffer(4)
        flag.zero()
        c.run([b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else []))
        hip.sync()
        outs.append(out.download(code))
    assert not np.any(outs[1] == code(0xFFFFFFFF if dt == "f32" else 0xFFFF)), "unwritten outputs"
    differ = np.count_nonzero(outs[0] != outs[1])
    assert differ == 0, f"{differ} of {outs[0].size} outputs differ from the four-wave tiles'"
