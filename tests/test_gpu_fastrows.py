"""FAST mode's row nests (wrows.hip) and functions (pk_expf_fast,
pk_erff_fast) on the device.

- The functions: the largest distance in units in the last place from the
  interpreter's musl-method expf and erff over every one of the 2^32 f32
  inputs (presk_hip_scalar_digest's ulp scans), held to the bounds the
  kernels' order names rely on (EXP_ULP, ERF_ULP).
- Row sums, means and `sum_to` onto rows: bit for bit the declared
  `lanes64xV-tree` order (oracle/lanes.py) at the configurations' shapes.
- Softmax (three passes, two, masked), cross entropy and its vjp: within a
  band of the float64 result of the same stored inputs -- the exponential's
  bound, the lane sum's (at most CH V + 6 additions of positive terms), the
  quotient's, and one rounding to the storage type -- with the masked
  positions exactly zero and every row's outputs summing to 1 within the
  same band; NaN, infinite and fully masked rows as the EXACT kernels give
  them."""
import ctypes

import numpy as np
import pytest

from oracle import cexec
from oracle.lanes import lanes_tree_sum
from presk_amd import hip
from presk_amd import lower as L
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand

EXP_ULP = 1         # pk_expf_fast against musl's expf, every f32 (measured: 1)
ERF_ULP = 3         # pk_erff_fast against musl's erff, every f32 (measured: 3)
U = 2.0 ** -24
HALF = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}   # half a unit, relative


@pytest.fixture(scope="module")
def ex():
    return hip.HipExec(0, mode=hip.FAST)


def scan(fn):
    d = ctypes.c_uint64()
    hip.check(hip.lib().presk_hip_scalar_digest(fn, 0, 1 << 32, ctypes.byref(d)))
    return d.value


@pytest.mark.parametrize("name,fn,bound", [("expf", 50, EXP_ULP), ("erff", 51, ERF_ULP)])
def test_fast_function_ulp_bound_over_every_f32(name, fn, bound):
    hip.init(0)
    worst = scan(fn)
    differ = scan(fn + 10)
    print(f"[fastfns] {name}: at most {worst} ulp from musl, {differ} of 2^32 inputs differ", flush=True)
    assert worst <= bound, worst
    assert differ > 0          # not musl itself


def run(ex, low, ins, mode_kind="rows"):
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    nb = k.output.numel * hip.STORAGE_BYTES[low.dtype]
    out = hip.DeviceBuffer(nb)
    out.upload(np.full(nb, 0xFF, np.uint8))
    c = ex.run(low.text, low.dtype, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert c.kind == mode_kind, c.kind
    return c, out.download(np.float32 if low.dtype == "f32" else np.uint16)


SUMS = [
    ("mean-course-ln", lambda dt: L.reduce_axis("mean", "model", [O(A(("batch", 64), ("seq", 256), ("model", 384)))], dt), "f32"),
    ("mean-mlp-ln", lambda dt: L.reduce_axis("mean", "model", [O(A(("batch", 8192), ("model", 768)))], dt), "bf16"),
    ("mean-llama-rms", lambda dt: L.reduce_axis("mean", "model", [O(A(("batch", 1), ("seq", 2048), ("model", 4096)))], dt), "bf16"),
    ("sum-vocab65", lambda dt: L.reduce_axis("sum", "vocab", [O(A(("batch", 7), ("seq", 60), ("vocab", 65)))], dt), "f32"),
    ("sum_to-rows", lambda dt: L.sum_to([O(A(("batch", 64), ("seq", 256), ("model", 384))), O(A(("batch", 64), ("seq", 256)))], dt), "f32"),
    ("mean-f16", lambda dt: L.reduce_axis("mean", "model", [O(A(("batch", 300), ("model", 1000)))], dt), "f16"),
    # 16-bit rows of at most 256 elements: blocks of 4 (8-byte loads)
    ("sum-bf16-256", lambda dt: L.reduce_axis("sum", "seq2", [O(A(("batch", 64), ("heads", 6), ("seq", 256), ("seq2", 256)))], dt), "bf16"),
    ("mean-f16-100", lambda dt: L.reduce_axis("mean", "model", [O(A(("batch", 300), ("model", 100)))], dt), "f16"),
]


@pytest.mark.parametrize("name,mk,dt", SUMS, ids=[s[0] for s in SUMS])
def test_fast_row_sums_are_the_declared_order(ex, name, mk, dt):
    low = mk(dt)
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    n = k.inputs[0].dims[-1]
    rows = k.inputs[0].numel // n
    rng = np.random.default_rng(7)
    x = fmt.roundtrip((rng.standard_normal((rows, n)) * np.exp2(rng.integers(-6, 6, (rows, n)))).astype(np.float32), dt)
    ins = [fmt.encode(x, dt)]
    if low.name == "sum_to":
        ins.append(fmt.encode(np.zeros(rows, np.float32), dt))      # the template operand (its shape only)
    c, got = run(ex, low, ins)
    vec = int(c.order.split("x")[1].split("-")[0])
    assert c.order == f"lanes64x{vec}-tree", c.order
    esz = 4 if dt == "f32" else 2
    # 16-byte blocks, 8-byte ones for 16-bit rows of at most 256, else single elements
    assert vec == (4 if esz == 2 and n <= 256 and n % 4 == 0 else 1 if (n * esz) % 16 else 16 // esz)
    s = lanes_tree_sum(x, vec)
    if low.name.startswith("mean"):
        s = (s / np.float32(n)).astype(np.float32)
    want = fmt.encode(s, dt)
    assert got.tobytes() == want.tobytes(), f"{name}: {np.count_nonzero(got != want)} of {rows} rows differ"


def softmax_cases():
    for dt in ("f32", "bf16"):
        s = O(A(("batch", 64), ("heads", 6), ("seq", 256), ("seq2", 256)))
        m = O(A(("seq", 256), ("seq2", 256)), "idx")
        yield f"course-masked-{dt}", L.masked_softmax("seq2", [s, m], dt), 256, True
        yield f"course-masked2-{dt}", L.masked_softmax("seq2", [s, m], dt, two_passes=True), 256, True
        s2 = O(A(("batch", 40), ("seq", 300)))
        yield f"softmax3-300-{dt}", L.softmax("seq", [s2], dt), None, False
        yield f"softmax2-300-{dt}", L.softmax_two_pass("seq", [s2], dt), None, False
    s = O(A(("batch", 1), ("heads", 32), ("seq", 2048), ("seq2", 2048)))
    m = O(A(("seq", 2048), ("seq2", 2048)), "idx")
    yield "llama-masked-bf16", L.masked_softmax("seq2", [s, m], "bf16"), 2048, True


def band(n, vec):
    """relative error of one output: the exponential's, the lane sums' (at
    most ceil(n / 64 / vec) vec + 6 additions of nonnegative terms), the
    quotient's (one and a half units), each at most 2u a unit"""
    nb = -(-n // vec)
    ch = -(-nb // 64)
    return 2 * U * (EXP_ULP + ch * vec + 6 + 2)


@pytest.mark.parametrize("case", list(softmax_cases()), ids=lambda c: c[0])
def test_fast_softmax_within_band(ex, case):
    name, low, T, masked = case
    dt = low.dtype
    from oracle import kernel_text as kt
    k = kt.parse_kernel(low.text)
    n = k.inputs[0].dims[-1]
    rows = k.inputs[0].numel // n
    print(f"[fastrows] {name}: {rows} rows of {n}", flush=True)
    rng = np.random.default_rng(9)
    x = fmt.roundtrip((rng.standard_normal((rows, n)) * 3).astype(np.float32), dt)
    ins = [fmt.encode(x, dt)]
    if masked:
        mask = np.tril(np.ones((T, T), np.int64))
        # a row the mask allows nowhere, and a second mask value above 1
        mask[5, :] = 0
        mask[7, 3] = 2
        ins.append(mask.ravel())
    c, raw = run(ex, low, ins)
    assert c.order.startswith("lanes64x") and c.order.endswith("-tree+fast-exp"), c.order
    vec = int(c.order.split("x")[1].split("-")[0])
    got = fmt.decode(raw, dt).reshape(rows, n).astype(np.float64)
    allowed = np.ones((rows, n), bool)
    if masked:
        allowed = (mask > 0)[np.arange(rows) % T]
    xv = np.where(allowed, x.astype(np.float64), -np.inf)
    mx = xv.max(axis=1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    e = np.where(allowed, np.exp(xv - mx), 0.0)
    z = e.sum(axis=1, keepdims=True)
    ref = np.divide(e, z, out=np.zeros_like(e), where=z > 0)
    assert np.all(got[~allowed] == 0.0), "masked positions"
    tol = band(n, vec) * ref + HALF[dt] * 2 * np.maximum(ref, np.abs(got)) + 2.0 ** -126
    err = np.abs(got - ref)
    assert np.all(err <= tol), f"{np.count_nonzero(err > tol)} outputs outside the band"
    live = allowed.any(axis=1)
    rs = got.sum(axis=1)
    # each output rounded once within half a unit of itself: the row's sum
    # within that of 1
    assert np.all(np.abs(rs[live] - 1) <= band(n, vec) + 4 * HALF[dt]), (rs[live].min(), rs[live].max())
    assert np.all(rs[~live] == 0)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fast_softmax_special_rows(ex, dt):
    """NaN first, NaN later, +inf, -inf and a fully masked row: the FAST
    kernel's NaN positions and zeros are the EXACT oracle's; every finite
    output of the other rows within the band"""
    T = 40
    s = O(A(("batch", 3), ("seq", T), ("seq2", T)))
    low = L.masked_softmax("seq2", [s, O(A(("seq", T), ("seq2", T)), "idx")], dt)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, T, T)).astype(np.float32)
    x[0, 10, 0] = np.nan
    x[0, 11, 6] = np.nan
    x[0, 12, 2] = np.inf
    x[1, 13, 1] = -np.inf
    x[2, 30, 35] = np.nan                    # disallowed: no effect
    mask = np.tril(np.ones((T, T), np.int64))
    mask[20] = 0
    ins = [fmt.encode(x, dt), mask.ravel()]
    want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
    c, raw = run(ex, low, ins)
    vec = int(c.order.split("x")[1].split("-")[0])
    got = fmt.decode(raw, dt).astype(np.float64)
    ref = fmt.decode(want, dt).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    allowed = np.broadcast_to(mask > 0, (3, T, T)).ravel()
    assert np.all(got[~allowed] == 0) and np.all(got[20 * T:21 * T] == 0)
    fin = np.isfinite(ref)
    assert np.all(np.abs(got[fin] - ref[fin]) <= band(T, vec) * np.abs(ref[fin]) + 4 * HALF[dt] * np.abs(ref[fin]) + 2.0 ** -126)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fast_cross_entropy_within_band(ex, dt):
    """the course's loss rows ([64, 256] tokens over V 65, single-element
    blocks) and the vjp: log(z) + m - x[y] and (e / z - onehot) ct against
    float64"""
    B, T, V = 64, 256, 65
    lg = O(A(("batch", B), ("seq", T), ("vocab", V)))
    ids = O(A(("batch", B), ("seq", T)), "idx")
    rows = O(A(("batch", B), ("seq", T)))
    rng = np.random.default_rng(4)
    x = fmt.roundtrip((rng.standard_normal((B * T, V)) * 2).astype(np.float32), dt)
    y = rng.integers(0, V, B * T).astype(np.int64)
    ct = fmt.roundtrip(np.full(B * T, 1.0 / (B * T), np.float32), dt)
    xd = x.astype(np.float64)
    m = xd.max(axis=1, keepdims=True)
    z = np.exp(xd - m).sum(axis=1)
    loss = np.log(z) + m[:, 0] - xd[np.arange(B * T), y]
    low = L.cross_entropy([lg, ids], dt)
    c, raw = run(ex, low, [fmt.encode(x, dt), y])
    assert c.order == "lanes64x1-tree+fast-exp", c.order
    got = fmt.decode(raw, dt).astype(np.float64)
    # log's argument carries the sum's relative error; the terms are O(|m|)
    tol = band(V, 1) * 4 * (np.abs(m[:, 0]) + np.abs(xd[np.arange(B * T), y]) + 1) + 2 * HALF[dt] * np.abs(loss)
    assert np.all(np.abs(got - loss) <= tol)
    low = L.cross_entropy_vjp([lg, ids, rows], dt)
    c, raw = run(ex, low, [fmt.encode(x, dt), y, fmt.encode(ct, dt)])
    got = fmt.decode(raw, dt).astype(np.float64).reshape(B * T, V)
    sm = np.exp(xd - m) / z[:, None]
    ref = (sm - (np.arange(V)[None, :] == y[:, None])) * ct.astype(np.float64)[:, None]
    tol = band(V, 1) * np.abs(sm * ct[:, None]) + 2 * HALF[dt] * np.abs(ref) + 2 * U * np.abs(ct[:, None]) + 2.0 ** -126
    assert np.all(np.abs(got - ref) <= tol)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fast_gelu_within_band(ex, dt):
    """config 2's GELU in FAST mode (erf by pk_erff_fast): within the erf
    bound, carried through x (1 + erf(x / sqrt 2)) / 2, of float64"""
    from scipy.special import erf
    low = L.unary("gelu", [O(A(("batch", 8192), 3072))], dt)
    rng = np.random.default_rng(6)
    x = fmt.roundtrip((rng.standard_normal((8192, 3072)) * 2).astype(np.float32), dt)
    c, raw = run(ex, low, [fmt.encode(x, dt)], "generic")
    assert c.order == "sequential+fast-exp-erf", c.order
    got = fmt.decode(raw, dt).astype(np.float64).reshape(x.shape)
    xd = x.astype(np.float64)
    ref = xd * (1 + erf(xd / np.sqrt(2))) / 2
    tol = np.abs(xd) * (ERF_ULP + 6) * 2 * U + 8 * U * np.abs(ref) + 2 * HALF[dt] * np.abs(ref) + 2.0 ** -126
    err = np.abs(got - ref)
    assert np.all(err <= tol), f"{np.count_nonzero(err > tol)} outside"
