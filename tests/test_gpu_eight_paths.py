"""The contractions that reach the f32 MFMA kernel through widened copies --
e8m15 storage (the codes widened exactly, the f32 sums narrowed with the
epilogue) and integer weights (f32(q) * s, crates/presk-rt/src/quant.rs:
248-252) -- at the sizes where the planner takes the eight-wave tiles: the
course step's [16384 x 384] . [384 x 384] (256 x 96 tiles), the Linear
module's [4096 x 1024] . [1024 x 1024] (128 x 128 tiles of eight waves) and
a weight gradient over K 16384 (eight-wave 128 x 128 tiles, split).  20 000
sampled outputs against the float64 product of the same loaded operands:
within two f32 orders of the same sums (2 gamma_K sum|x_k w_k|) plus one
unit of the storage type for the sum and for the result, the bulk far inside
it (median below 1/16 of the band), every output written."""
import numpy as np
import pytest

from presk_amd import hip
from presk_amd import lower as L
from presk_amd import quant as Q
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand
UNIT = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10, "e8m15": 2.0 ** -15}
SHAPES = {"course": (16384, 384, 384), "linear": (4096, 1024, 1024)}


def band_check(a, b, got, what, rng, dt, transpose_a=False):
    """a: [M, K] (or [K, M] when transpose_a), b: [K, N], got: [M, N]."""
    M, N = got.shape
    assert np.all(np.isfinite(got)), f"{what}: unwritten or non-finite outputs"
    ms, ns = rng.integers(0, M, 20000), rng.integers(0, N, 20000)
    exact, S = np.empty(len(ms)), np.empty(len(ms))
    for c0 in range(0, len(ms), 2000):
        rows = (a[:, ms[c0:c0 + 2000]].T if transpose_a else a[ms[c0:c0 + 2000]]).astype(np.float64)
        cols = b[:, ns[c0:c0 + 2000]].T.astype(np.float64)
        exact[c0:c0 + 2000] = np.einsum("ik,ik->i", rows, cols)
        S[c0:c0 + 2000] = np.einsum("ik,ik->i", np.abs(rows), np.abs(cols))
    K = a.shape[0] if transpose_a else a.shape[1]
    g = got[ms, ns].astype(np.float64)
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    bound = 2 * gamma * S + UNIT[dt] * (S + 2 * np.maximum(np.abs(exact), np.abs(g))) + 1e-30
    err = np.abs(g - exact)
    assert np.all(err <= bound), f"{what}: {np.count_nonzero(err > bound)} sampled elements outside the band"
    assert np.median(err / bound) < 1 / 16, f"{what}: median error {np.median(err / bound):.3g} of the band"


@pytest.mark.parametrize("shape", list(SHAPES))
def test_e8m15_on_eight_wave_tiles(shape):
    M, K, N = SHAPES[shape]
    dt = "e8m15"
    print(f"[eight] e8m15 {shape}", flush=True)
    rng = np.random.default_rng(21)
    x = fmt.roundtrip(rng.standard_normal((M, K), dtype=np.float32), dt)
    w = fmt.roundtrip(rng.standard_normal((K, N), dtype=np.float32), dt)
    low = L.dot([O(A(("batch", M), K)), O(A(K, N))], dt)
    c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
    assert c.kind == "gemm" and c.order == "mfma-f32-k4", (c.kind, c.order)
    ins = [hip.DeviceBuffer.of(fmt.encode(v, dt)) for v in (x, w)]
    out = hip.DeviceBuffer(M * N * 3)
    out.upload(np.full(M * N * 3, 0xFF, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    c.run([b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else []))
    hip.sync()
    got = fmt.decode(out.download(np.uint8), dt).reshape(M, N)
    band_check(x, w, got, f"e8m15 {shape}", rng, dt)


@pytest.mark.parametrize("shape,bits,dt", [("course", 8, "f32"), ("linear", 8, "f32"), ("course", 4, "bf16"),
                                           ("linear", 8, "bf16")])
def test_integer_weights_on_eight_wave_tiles(shape, bits, dt):
    M, K, N = SHAPES[shape]
    print(f"[eight] int{bits} {dt} {shape}", flush=True)
    rng = np.random.default_rng(22 + bits)
    x = fmt.roundtrip(rng.standard_normal((M, K), dtype=np.float32), dt)
    qt = Q.quantize(rng.standard_normal((K, N)), (K, N), Q.Quant(bits, 0))
    low = L.dot([O(A(("batch", M), K)), O(A(K, N))], dt)
    text = Q.mark(low.text, 1, Q.of_quant(qt, (K, N)))
    c = hip.Compiled(text, dt, low.lanes, hip.FAST)
    assert c.kind == "gemm" and c.order == "mfma-f32-k4", (c.kind, c.order)
    bx, bq, bs = hip.DeviceBuffer.of(fmt.encode(x, dt)), hip.DeviceBuffer.of(qt.data), hip.DeviceBuffer.of(qt.scales)
    nb = M * N * hip.STORAGE_BYTES[dt]
    out = hip.DeviceBuffer(nb)
    out.upload(np.full(nb, 0xFF, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    c.run([bx.ptr, bq.ptr, out.ptr, bs.ptr] + ([flag.ptr] if c.guarded else []))
    hip.sync()
    got = fmt.decode(out.download(np.float32 if dt == "f32" else np.uint16), dt).reshape(M, N)
    wv = qt.dequantize().astype(np.float32).reshape(K, N)
    band_check(x, wv, got, f"int{bits} {dt} {shape}", rng, dt)


def test_e8m15_weight_gradient_on_eight_wave_split_tiles():
    # [16384 x 384]^T . [16384 x 384]: split K over eight-wave 128 x 128 tiles
    dt = "e8m15"
    print("[eight] e8m15 weight gradient", flush=True)
    rng = np.random.default_rng(23)
    T, M, N = 16384, 384, 384
    x = fmt.roundtrip(rng.standard_normal((T, M), dtype=np.float32), dt)
    dy = fmt.roundtrip((rng.standard_normal((T, N)) / 16384).astype(np.float32), dt)
    low = L.dot_vjp_r([O(A(("batch", 64), ("seq", 256), M)), O(A(("batch", 64), ("seq", 256), N))], dt)
    c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
    assert c.kind == "gemm" and c.order.startswith("mfma-f32-k4-split"), (c.kind, c.order)
    ins = [hip.DeviceBuffer.of(fmt.encode(v, dt)) for v in (x, dy)]
    out = hip.DeviceBuffer(M * N * 3)
    out.upload(np.full(M * N * 3, 0xFF, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    c.run([b.ptr for b in ins] + [out.ptr] + ([flag.ptr] if c.guarded else []))
    hip.sync()
    got = fmt.decode(out.download(np.uint8), dt).reshape(M, N)
    band_check(x, dy, got, "e8m15 weight gradient", rng, dt, transpose_a=True)
