"""The lowering restatement (presk_amd/lower.py) against the reference's own
kernel-text snapshots: Linear{3,2} at batch 4 in f32
(crates/presk-kernel/tests/snapshots/conformance__linear_kernels.snap) and
Linear{4,8} at batch 2 in f64, f32, bf16, f16, e8m15
(crates/presk-export-c/tests/snapshots/kernels__linear_c.snap)."""
import os

from presk_amd import lower as L

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _split(text):
    out, cur = [], []
    for line in text.split("\n"):
        if line.startswith("kernel "):
            cur = [line]
        elif cur:
            cur.append(line)
            if line == "}":
                out.append("\n".join(cur) + "\n")
                cur = []
    return out


def linear(batch, n_in, n_out, dtype):
    x = L.Operand(L.ax(("batch", batch), n_in))
    w = L.Operand(L.ax(n_in, n_out))
    b = L.Operand(L.ax(n_out))
    d = L.dot([x, w], dtype)
    a = L.elementwise_binary("add", [L.Operand(d.out_axes), b], dtype)
    return [d.text, a.text]


def test_linear_f32_snapshot():
    snap = _split(open(os.path.join(GOLD, "conformance__linear_kernels.snap")).read())
    assert linear(4, 3, 2, "f32") == snap


def test_linear_c_snapshot_all_types():
    text = open(os.path.join(GOLD, "kernels__linear_c.snap")).read()
    lines = [ln[3:] if ln.startswith("// ") else ln[2:] for ln in text.split("\n") if ln.startswith("//")]
    snap = _split("\n".join(lines))
    got = []
    for dt in ("f64", "f32", "bf16", "f16", "e8m15"):
        got += linear(2, 4, 8, dt)
    assert got == snap


def test_num_prints_like_rust():
    assert L.num(1.0) == "1"
    assert L.num(0.5) == "0.5"
    assert L.num(1e-5) == "0.00001"
    assert L.num(L.SQRT_2) == "1.4142135623730951"
    assert L.num(-1) == "-1"
    assert L.num(float("inf")) == "inf"
