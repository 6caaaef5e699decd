"""The contraction plans the course step actually runs, at their real sizes,
against the float64 product of the same rounded operands.

The weight gradients of config 4 (`dot_vjp_r`, `lower.rs:555-584`) sum over
batch x seq = 16 384 terms into a few output tiles, so the planner splits K
across workgroups and a second kernel adds the partials in split order.
Each plan below is the one the bench's step takes (its order string names
the split); every output element is compared with the exact product within
2 gamma_K sum|x_k w_k| plus one unit of the storage type for the sum and for
the result, and the bulk must lie far inside that band, so a lost or doubled
k-range or a misplaced partial cannot pass.

Also the e8m15 `dot+add` whose K is split (the bias is added after the
first narrowing by the e8m15 plan's own last kernel, not by the partials'
reduction)."""
import numpy as np
import pytest

from oracle import cexec
from presk_amd import hip
from presk_amd import lower as L
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand

ULP = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10, "e8m15": 2.0 ** -15}
B, T = 64, 256


def vjp_r(n_x, n_ct, dt):
    return L.dot_vjp_r([O(A(("batch", B), ("seq", T), n_x)), O(A(("batch", B), ("seq", T), n_ct))], dt)


# (name, lowering, storage type, the split the plan must take)
PLANS = [
    ("attn-proj-384x384", lambda dt: vjp_r(384, 384, dt), "f32", 28),
    ("attn-proj-384x384", lambda dt: vjp_r(384, 384, dt), "bf16", 14),
    ("head-384x65", lambda dt: vjp_r(384, 65, dt), "f32", 64),
    ("head-384x65", lambda dt: vjp_r(384, 65, dt), "bf16", 64),
    ("mlp-up-384x1536", lambda dt: vjp_r(384, 1536, dt), "f32", 7),
    ("mlp-up-384x1536", lambda dt: vjp_r(384, 1536, dt), "bf16", 7),
    ("mlp-down-1536x384", lambda dt: vjp_r(1536, 384, dt), "f32", 7),
    ("mlp-down-1536x384", lambda dt: vjp_r(1536, 384, dt), "bf16", 7),
]


@pytest.fixture(scope="module")
def ex():
    return hip.HipExec(0, mode=hip.FAST)


def band_check(got, exact, S, K, dt, what):
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    bound = 2 * gamma * S + ULP[dt] * (S + 2 * np.maximum(np.abs(exact), np.abs(got))) + 1e-30
    err = np.abs(got - exact)
    assert np.all(np.isfinite(got)), f"{what}: unwritten or non-finite outputs"
    assert np.all(err <= bound), f"{what}: {np.count_nonzero(err > bound)} of {err.size} elements outside the band"
    assert np.median(err / bound) < 1 / 64, f"{what}: median error {np.median(err / bound):.3g} of the band"


@pytest.mark.parametrize("name,mk,dt,split", PLANS, ids=lambda v: v if isinstance(v, (str, int)) else "")
def test_weight_gradient_plan_within_band(ex, name, mk, dt, split):
    from oracle import kernel_text as kt
    low = mk(dt)
    k = kt.parse_kernel(low.text)
    print(f"[plans] {name} {dt} split {split}", flush=True)
    rng = np.random.default_rng(11)
    # activations ~N(0,1), cotangents at the scale of a mean loss's (1/16384)
    vals = [fmt.roundtrip(rng.standard_normal(k.inputs[0].dims, dtype=np.float32), dt),
            fmt.roundtrip((rng.standard_normal(k.inputs[1].dims, dtype=np.float32) / 16384).astype(np.float32), dt)]
    nb = k.output.numel * hip.STORAGE_BYTES[dt]
    out = hip.DeviceBuffer(nb)
    out.upload(np.full(nb, 0xFF, np.uint8))
    c = ex.run(low.text, dt, [hip.DeviceBuffer.of(fmt.encode(v, dt)) for v in vals], out, lanes=low.lanes)
    assert c.kind == "gemm", c.kind
    assert c.order.endswith(f"-split{split}"), f"the plan is {c.order}, not split {split}"
    raw = out.download(np.float32 if dt == "f32" else np.uint16)
    got = fmt.decode(raw, dt).astype(np.float64).reshape(k.output.dims)
    a = vals[0].reshape(B * T, -1).astype(np.float64)
    b = vals[1].reshape(B * T, -1).astype(np.float64)
    exact = a.T @ b
    S = np.abs(a).T @ np.abs(b)
    band_check(got, exact, S, B * T, dt, f"{name} {dt} [{c.order}]")


def test_e8m15_bias_with_split_k(ex):
    """x[64,1024] . w[1024,1024] + b in e8m15: few rows and a long K, so K is
    split; the partials' reduction must not read the bias (the e8m15 plan
    passes none there) and the result must equal the oracle's within the band."""
    from oracle import kernel_text as kt
    dt = "e8m15"
    x, w = O(A(("batch", 64), 1024)), O(A(1024, 1024))
    d = L.dot([x, w], dt)
    low = L.dot([x, w, O(A(1024))], dt, epilogue=(True, d.out_axes))
    k = kt.parse_kernel(low.text)
    rng = np.random.default_rng(12)
    vals = [fmt.roundtrip(rng.standard_normal(bf.dims).astype(np.float32), dt) for bf in k.inputs]
    ins = [fmt.encode(v, dt) for v in vals]
    want, _ = cexec.run(low.text, dt, ins, lanes=low.lanes)
    nb = k.output.numel * 3
    out = hip.DeviceBuffer(nb)
    out.upload(np.full(nb, 0xFF, np.uint8))
    c = ex.run(low.text, dt, [hip.DeviceBuffer.of(a) for a in ins], out, lanes=low.lanes)
    assert c.kind == "gemm" and "-split" in c.order, (c.kind, c.order)
    got = fmt.decode(out.download(want.dtype), dt).astype(np.float64).reshape(64, 1024)
    ref = fmt.decode(want, dt).astype(np.float64).reshape(64, 1024)
    xa = vals[0].reshape(64, 1024).astype(np.float64)
    wa = vals[1].reshape(1024, 1024).astype(np.float64)
    S = np.abs(xa) @ np.abs(wa)
    K = 1024
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    bound = 2 * gamma * S + ULP[dt] * (S + 2 * np.maximum(np.abs(ref), np.abs(got))) + 1e-30
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound), f"{np.count_nonzero(err > bound)} elements outside the band [{c.order}]"
    assert np.median(err / bound) < 1 / 64
