"""The oracle's reader of PSK-Kernel text, pinned by the reference's own
snapshots (crates/presk-kernel/tests/snapshots/conformance__linear_kernels.snap,
crates/presk-export-c/tests/snapshots/kernels__linear_c.snap, copied as
fixtures under tests/golden/), and its C printer's semantics on them."""
import os

import numpy as np

from oracle import cexec
from tests import fmt
from oracle import kernel_text as kt

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def snapshot_kernels():
    ks = kt.split_kernels(open(os.path.join(GOLD, "conformance__linear_kernels.snap")).read())
    c = open(os.path.join(GOLD, "kernels__linear_c.snap")).read()
    lines = [ln[3:] if ln.startswith("// ") else ln[2:] for ln in c.split("\n") if ln.startswith("//")]
    return ks + kt.split_kernels("\n".join(lines))


def test_snapshots_round_trip():
    ks = snapshot_kernels()
    assert len(ks) == 12
    for text in ks:
        assert kt.show_kernel(kt.parse_kernel(text)) == text


def _seq_dot(x, w, dt):
    out = np.zeros((x.shape[0], w.shape[1]), dtype=dt)
    for i in range(x.shape[0]):
        for j in range(w.shape[1]):
            s = dt(0)
            for k in range(x.shape[1]):
                s = dt(s + dt(x[i, k] * w[k, j]))
            out[i, j] = s
    return out


def test_snapshot_kernels_compute_sequential_dot():
    """Every snapshot `dot` (row-wise, blocked, vector lanes; f64, f32, bf16,
    f16, e8m15) gives the in-order sum in the arithmetic type rounded once to
    the storage type, and every `add` the broadcast sum, bit for bit."""
    rng = np.random.default_rng(0)
    for text in snapshot_kernels():
        k = kt.parse_kernel(text)
        ty = k.output.ty
        dt = np.float64 if ty == "f64" else np.float32
        vals = [fmt.roundtrip(rng.standard_normal(b.dims).astype(np.float32), ty).astype(dt) for b in k.inputs]
        lanes = (2 if ty == "f64" else 4) if k.nvec else 1
        out, flag = cexec.run(text, ty, [fmt.encode(v, ty) if ty != "f64" else v.ravel() for v in vals], lanes=lanes)
        got = fmt.decode(out, ty).reshape(k.output.dims)
        exact = _seq_dot(*vals, dt) if k.name == "dot" else (vals[0] + vals[1]).astype(dt)
        want = exact if ty == "f64" else fmt.roundtrip(exact.astype(np.float32), ty)
        assert np.array_equal(got, want), (k.name, ty)
        assert not flag
