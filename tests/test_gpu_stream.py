"""The streamed-panel contraction (gemm.hip's stream_kernel: a 128-row panel
of A kept in LDS, B's 64-column tiles streamed across it) for products with
K of at most two k-blocks, the attention's scores.  It computes each output
with the same MFMAs (32x32x16 in 16-bit storage, 16x16x4 in f32) over the
same k-steps as the 128 x 64 tiles' kernel, so the two must agree bit for
bit; the tiles' kernel is the one the plan takes under
PRESK_HIP_GEMM_TILE=128x64.  Both
are also held to the oracle's band on sampled rows (as tests/test_gpu_gemm.py
bounds a reassociated sum)."""
import os

import numpy as np
import pytest

from presk_amd import hip
from presk_amd import lower as L
from tests import fmt

pytestmark = pytest.mark.gpu
A, O = L.ax, L.Operand

UNIT = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11, "f32": 2.0 ** -24}
ESZ = {"bf16": 2, "f16": 2, "f32": 4}


def scores(dt, B, H, T, T2, HD):
    q = O(A(("batch", B), ("heads", H), ("seq", T), ("hd", HD)))
    k = O(A(("batch", B), ("heads", H), ("seq2", T2), ("hd", HD)))
    return L.ein([q, k], [["batch", "heads", "seq", "hd"], ["batch", "heads", "seq2", "hd"]],
                 ["batch", "heads", "seq", "seq2"], dt)


CASES = [
    ("llama-scores-bf16", "bf16", (1, 32, 2048, 2048, 128), 1.0),
    ("course-scores-bf16", "bf16", (64, 6, 256, 256, 64), 1.0),
    ("course-scores-f16", "f16", (64, 6, 256, 256, 64), 1.0),
    # few panels: each panel's columns split into runs (items fill the CUs)
    ("few-panels-bf16", "bf16", (1, 2, 256, 2048, 128), 1.0),
    # sums past f16's range: infinities and the overflow flag, as the tiles give them
    ("overflow-f16", "f16", (2, 2, 128, 256, 128), 40.0),
    # f32 (k-blocks of 32): the course's scores (K 64, the headline's), and K 32
    ("course-scores-f32", "f32", (64, 6, 256, 256, 64), 1.0),
    ("k32-f32", "f32", (2, 4, 256, 512, 32), 1.0),
]


def run(low, ins, tile):
    if tile:
        os.environ["PRESK_HIP_GEMM_TILE"] = tile
    else:
        os.environ.pop("PRESK_HIP_GEMM_TILE", None)
    try:
        c = hip.Compiled(low.text, low.dtype, low.lanes, hip.FAST)
    finally:
        os.environ.pop("PRESK_HIP_GEMM_TILE", None)
    assert c.kind == "gemm" and c.order == ("mfma-f32-k4" if low.dtype == "f32" else "mfma-k16"), (c.kind, c.order)
    bufs = [hip.DeviceBuffer.of(a) for a in ins]
    n_out = 1
    for a in low.out_axes:
        n_out *= a.len
    esz = ESZ[low.dtype]
    out = hip.DeviceBuffer(esz * n_out)
    out.upload(np.full(esz * n_out, 0xFF, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    ptrs = [b.ptr for b in bufs] + [out.ptr] + ([flag.ptr] if c.guarded else [])
    c.run(ptrs)
    hip.sync()
    f = int(flag.download(np.uint32)[0]) if c.guarded else 0
    return out.download(np.uint16 if esz == 2 else np.float32), f


@pytest.mark.parametrize("name,dt,shape,scale", CASES, ids=[c[0] for c in CASES])
def test_streamed_panels_equal_the_tiles(name, dt, shape, scale):
    hip.init(0)
    B, H, T, T2, HD = shape
    print(f"[stream] {name}: {B}x{H} of {T}x{T2}, K {HD}", flush=True)
    low = scores(dt, B, H, T, T2, HD)
    rng = np.random.default_rng(11)
    q = fmt.roundtrip((rng.standard_normal((B, H, T, HD)) * scale).astype(np.float32), dt)
    k = fmt.roundtrip((rng.standard_normal((B, H, T2, HD)) * scale).astype(np.float32), dt)
    ins = [fmt.encode(q, dt), fmt.encode(k, dt)]
    got, f_got = run(low, ins, None)
    want, f_want = run(low, ins, "128x64")
    assert f_got == f_want
    bits = np.uint16 if dt != "f32" else np.uint32
    differ = np.count_nonzero(got.view(bits) != want.view(bits))
    assert differ == 0, f"{differ} of {got.size} outputs differ from the 128 x 64 tiles'"
    # the band of a reassociated sum on sampled rows, against float64
    out = fmt.decode(got, dt).astype(np.float64).reshape(B, H, T, T2)
    qd, kd = q.astype(np.float64), k.astype(np.float64)
    for b, h, t in ((0, 0, 0), (B - 1, H - 1, T - 1), (0, H // 2, T // 3)):
        ref = kd[b, h] @ qd[b, h, t]
        mag = np.abs(kd[b, h]) @ np.abs(qd[b, h, t])
        gamma = HD * 2.0 ** -24 / (1 - HD * 2.0 ** -24)
        fin = np.isfinite(out[b, h, t])
        tol = 2 * gamma * mag + UNIT[dt] * np.maximum(np.abs(ref), mag * 2.0 ** -10)
        assert np.all(np.abs(out[b, h, t][fin] - ref[fin]) <= tol[fin] + 1e-30)
    if name.startswith("overflow"):
        assert f_got == 1 and not np.all(np.isfinite(out))
