"""`.psk.d` leaves decoded on the device (presk_hip_pskd_decode,
presk_hip_pskd_decode_idx) against the oracle's decode (oracle/convert.c),
bytes and overflow guard identical: every code of the 4-, 8- and 16-bit
formats and random codes of wider ones, into every storage type; index
leaves of each width; the reference's data files through the reader; a
`params` file straight into a program's buffers; a description that is no
format refused."""
import ctypes
import os
import types

import numpy as np
import pytest

from presk_amd import hip, pskd
from presk_amd.pskd import Layout, Leaf

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pskd")
TO = {"f64": (0, 8), "f32": (1, 4), "bf16": (2, 2), "f16": (4, 2), "e8m15": (5, 3)}


@pytest.fixture(scope="module")
def lib(oracle_lib):
    L = oracle_lib
    L.po_pskd_decode.restype = ctypes.c_uint32
    L.po_pskd_decode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_size_t]
    L.po_pskd_idx.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    hip.init(0)
    return L


def code_bytes(codes: np.ndarray, width: int) -> np.ndarray:
    src = np.zeros(codes.size * width, np.uint8)
    for b in range(width):
        src[b::width] = (codes >> np.uint64(8 * b)).astype(np.uint8)
    return src


def device(src: np.ndarray, enc: pskd.Enc, n: int, to: str):
    code, nb = TO[to]
    s = hip.DeviceBuffer.of(src)
    d = hip.DeviceBuffer(n * nb)
    d.upload(np.full(n * nb, 0xA5, np.uint8))
    flag = hip.DeviceBuffer(4)
    flag.zero()
    desc = ctypes.create_string_buffer(enc.format.description(), 6) if enc.code == 3 else None
    hip.check(hip.lib().presk_hip_pskd_decode(s.ptr, enc.code, desc, n, d.ptr, to.encode(), flag.ptr, None))
    hip.sync()
    return d.download(np.uint8), int(flag.download(np.uint32, 1)[0])


def oracle(lib, src: np.ndarray, enc: pskd.Enc, n: int, to: str):
    code, nb = TO[to]
    out = np.zeros(n * nb, np.uint8)
    f = enc.format
    g = lib.po_pskd_decode(out.ctypes.data, code, src.ctypes.data, enc.code, f.width, f.p, f.emin, f.emax,
                           int(f.subnormals), pskd.SPECIALS.index(f.specials), n)
    return out, int(g)


def cases():
    rng = np.random.default_rng(17)
    out = []
    for name, f in [("e4m3", pskd.E4M3_SATURATING), ("e4m3fn", pskd.E4M3FN), ("e5m2", pskd.E5M2), ("e2m1", pskd.E2M1),
                    ("f16-described", pskd.F16)]:
        out.append((name, pskd.Enc(3, f), np.arange(1 << f.bits, dtype=np.uint64)))
    for name, f in [("p20-wide-range", pskd.Format(20, -254, 255)), ("p40-7-bytes", pskd.Format(40, -510, 511)),
                    ("p6-no-subnormals", pskd.Format(6, -30, 32, subnormals=False, specials="nan", overflow="nan"))]:
        f.check()
        out.append((name, pskd.Enc(3, f), rng.integers(0, 1 << min(f.bits, 63), 100_000, dtype=np.uint64)))
    out.append(("bf16", pskd.ENC_BF16, np.arange(1 << 16, dtype=np.uint64)))
    out.append(("f32", pskd.ENC_F32, rng.integers(0, 1 << 32, 100_000, dtype=np.uint64)))
    out.append(("f64", pskd.ENC_F64, np.concatenate([rng.integers(0, 2 ** 63, 50_000, dtype=np.uint64),
                                                     (rng.standard_normal(50_000) * 1e3).view(np.uint64)])))
    return out


@pytest.mark.parametrize("to", list(TO))
@pytest.mark.parametrize("case", cases(), ids=lambda c: c[0])
def test_leaf_decode_matches_oracle(lib, case, to):
    name, enc, codes = case
    print(f"[pskd] {name} -> {to}", flush=True)
    src = code_bytes(codes, enc.width)
    got, gf = device(src, enc, codes.size, to)
    want, wf = oracle(lib, src, enc, codes.size, to)
    assert gf == wf
    if got.tobytes() != want.tobytes():
        w = TO[to][1]
        bad = np.nonzero((got.reshape(-1, w) != want.reshape(-1, w)).any(axis=1))[0]
        pytest.fail(f"{name}->{to}: {bad.size} elements differ, first codes {[hex(int(c)) for c in codes[bad[:4]]]}")


@pytest.mark.parametrize("bound", [200, 60_000, 1 << 32, 1 << 40])
def test_idx_leaf_matches_oracle(lib, bound):
    rng = np.random.default_rng(bound % 1000)
    w = pskd.idx_width(bound)
    v = rng.integers(0, bound, 10_007, dtype=np.uint64)
    src = code_bytes(v, w)
    s = hip.DeviceBuffer.of(src)
    d = hip.DeviceBuffer(8 * v.size)
    hip.check(hip.lib().presk_hip_pskd_decode_idx(s.ptr, bound, v.size, d.ptr, None))
    hip.sync()
    want = np.zeros(v.size, np.int64)
    lib.po_pskd_idx(want.ctypes.data, src.ctypes.data, w, v.size)
    assert np.array_equal(d.download(np.int64), want) and np.array_equal(want.view(np.uint64), v)


def test_reference_files_through_the_reader(lib):
    for name in ("windows.psk.d", "tokens.psk.d", "pairs.psk.d", "reg.psk.d"):
        r = pskd.Reader(os.path.join(GOLD, name))
        got = r.load("f32")
        for i, ((buf, ty, ovf), leaf, raw) in enumerate(zip(got, r.layout.leaves(), r.leaf_bytes())):
            if leaf.bound is not None:
                want = np.zeros(raw.size // leaf.width, np.int64)
                lib.po_pskd_idx(want.ctypes.data, raw.ctypes.data, leaf.width, want.size)
                assert ty == "i64" and np.array_equal(buf.download(np.int64), want), (name, i)
            else:
                want, _ = oracle(lib, raw, r.header.encoding(i), raw.size // 8, "f32")
                assert ty == "f32" and buf.download(np.uint8).tobytes() == want.tobytes(), (name, i)


def test_params_file_into_program_buffers(lib, tmp_path):
    """A parameter tree written at e4m3 and bf16 loaded straight into a
    program's declared inputs (bf16 and f32 storage)."""
    from presk_amd.program import Buffers
    rng = np.random.default_rng(3)
    w = [pskd.E4M3_SATURATING.decode(int(c)) for c in rng.integers(0, 256, 64 * 48)]
    b = [pskd.BF16.decode(int(c)) for c in rng.integers(0x3C00, 0x4200, 48)]     # finite bf16 numbers, 2^-7 to 32
    layout = Layout.record([("w", Leaf((64, 48))), ("b", Leaf((48,)))])
    p = str(tmp_path / "theta.psk.d")
    pskd.write(p, "params Dense{64, 48}", layout, [[w, b]], [pskd.Enc.of(pskd.E4M3_SATURATING), pskd.ENC_BF16])
    prog = types.SimpleNamespace(bufs=Buffers())
    prog.bufs.alloc("w", "bf16", 64 * 48)
    prog.bufs.alloc("b", "f32", 48)
    pskd.load_params(prog, p, layout)
    got_w = prog.bufs.dev["w"].download(np.uint16)
    want_w = np.array([pskd.BF16.encode(x) for x in w], np.uint16)      # every e4m3 number is a bf16 number
    assert np.array_equal(got_w, want_w)
    assert np.array_equal(prog.bufs.dev["b"].download(np.float32), np.array(b, np.float32))


@pytest.mark.parametrize("model", ["gpt", "llama"])
def test_reference_checkpoint_into_stacked_buffers(lib, tmp_path, model):
    """A `params GPT` / `params Llama` file in the reference's tree (Block's
    leaves stacked over the layers, f32 and bf16 leaves) decoded into the
    program: each stacked leaf lands in the one buffer its layers' inputs
    are views of."""
    from presk_amd import gpt, llama
    from presk_amd.program import numel
    mod = gpt if model == "gpt" else llama
    s = mod.TINY
    layout, rename = mod.params_layout(s)
    rng = np.random.default_rng(9)
    encs = [pskd.ENC_BF16 if i % 3 == 1 else pskd.ENC_F32 for i in range(len(layout.leaves()))]
    values = []
    for l, e in zip(layout.leaves(), encs):
        v = (rng.standard_normal(l.numel) * 0.02).astype(np.float32).astype(np.float64)
        if e is pskd.ENC_BF16:                          # the writer takes numbers of the leaf's format only
            u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
            u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)    # nearest even bf16
            v = u.view(np.float32).astype(np.float64)
        values.append(list(v))
    path = str(tmp_path / "theta.psk.d")
    pskd.write(path, "params GPT" if model == "gpt" else "params Llama", layout, [values], encs)
    prog = gpt.build(s, "f32", train=False)[0] if model == "gpt" else llama.build(s, "f32")[0]
    for n, axes in mod.param_shapes(s).items():          # the program's parameter inputs, declared
        prog.declare(n, "f32", numel(axes))
    pskd.load_params(prog, path, layout, rename=rename)
    leaves = gpt.opt_leaves(s) if model == "gpt" else llama.leaves(s)
    for i, (name, (axes, members)) in enumerate(leaves.items()):
        want = np.array(values[i], np.float64).astype(np.float32)
        if members is None:
            assert np.array_equal(prog.bufs.dev[name].download(np.float32), want), name
            continue
        per = numel(axes[1:])
        for l, m in enumerate(members):
            assert prog.bufs.dev[m].ptr == prog.bufs.dev[name].ptr + 4 * l * per     # a view of the stacked leaf
            got = prog.bufs.dev[m].download(np.float32)
            assert np.array_equal(got, want[l * per:(l + 1) * per]), (name, l)


def test_description_that_is_no_format_is_refused(lib):
    s = hip.DeviceBuffer(16)
    d = hip.DeviceBuffer(16)
    bad = ctypes.create_string_buffer(bytes([4, 0xFA, 0xFF, 8, 0, 0x80]), 6)      # flag bit 7
    rc = hip.lib().presk_hip_pskd_decode(s.ptr, 3, bad, 4, d.ptr, b"f32", None, None)
    assert rc != 0 and b"E9002" in hip.lib().presk_hip_last_error()
    odd = ctypes.create_string_buffer(bytes([4, 0xFA, 0xFF, 9, 0, 4]), 6)       # 17 exponent codes: no field
    assert hip.lib().presk_hip_pskd_decode(s.ptr, 3, odd, 4, d.ptr, b"f32", None, None) != 0
