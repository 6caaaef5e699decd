"""The .psk.d container's host logic (presk_amd/pskd.py) on the reference's
own cases (crates/presk-data/tests/data.rs) and data files: layouts from
types, idx widths, the headers of versions 1-3 and their byte counts, values
refused at write time, malformed files, and `params` files that need the
program's layout.  Leaf values are read back with the
oracle's decode (the device path is tests/test_gpu_pskd.py).

Data files (tests/golden/pskd/) are the reference's examples, copied as data:
examples/tests/data/windows.psk.d, examples/spec/minigpt/data/tokens.psk.d,
examples/tutorial/data/pairs.psk.d, examples/tests/train/reg.psk.d.  The
first two samples of windows.psk.d are the reference's info snapshot
(crates/presk-data/tests/snapshots/data__info_snapshot.snap)."""
import ctypes
import math
import os
import struct

import numpy as np
import pytest

from presk_amd import pskd
from presk_amd.pskd import DataError, Layout, Leaf

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pskd")


def code_of(fn):
    with pytest.raises(DataError) as e:
        fn()
    return e.value.code


def test_layouts_from_types():
    l = Layout.from_type_text("(idx[64][seq: 8], idx[64][seq: 8])")
    assert l == Layout(items=[Layout(Leaf((8,), 64)), Layout(Leaf((8,), 64))])
    assert l.sample_bytes() == 16
    assert Layout.from_type_text("ℝ[batch: 2, model: 4]").sample_bytes() == 64
    assert Layout.from_type_text("Real[3]").sample_bytes() == 24
    assert Layout.from_type_text("ℝ[]").sample_bytes() == 8
    assert Layout.from_type_text("(ℝ[model: 2], idx[10][])").leaves() == [Leaf((2,)), Leaf((), 10)]
    for bad in ["ℝ[..., 4]", "ℝ[D]", "idx[0][2]", "params MiniGPT", "nat", "ℝ[4] ℝ[4]", "(("]:
        assert code_of(lambda: Layout.from_type_text(bad)) == "E9001", bad


def test_idx_widths():
    assert [pskd.idx_width(b) for b in (1, 256, 257, 65_536, 65_537, 1 << 40)] == [1, 1, 2, 2, 4, 8]


def read_leaves(r: pskd.Reader, oracle_lib, first=0, count=None):
    """Each leaf's values through the oracle's decode, as f64 / i64 arrays."""
    L = oracle_lib
    L.po_pskd_decode.restype = ctypes.c_uint32
    L.po_pskd_decode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_size_t]
    L.po_pskd_idx.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    out = []
    for i, (leaf, raw) in enumerate(zip(r.layout.leaves(), r.leaf_bytes(first, count))):
        if leaf.bound is not None:
            n = raw.size // leaf.width
            v = np.zeros(n, np.int64)
            L.po_pskd_idx(v.ctypes.data, raw.ctypes.data, leaf.width, n)
        else:
            e = r.header.encoding(i)
            n = raw.size // e.width
            v = np.zeros(n, np.float64)
            f = e.format
            L.po_pskd_decode(v.ctypes.data, 0, raw.ctypes.data, e.code, f.width, f.p, f.emin, f.emax, int(f.subnormals),
                             pskd.SPECIALS.index(f.specials), n)
        out.append(v)
    return out


def test_reference_data_files(oracle_lib):
    r = pskd.Reader(os.path.join(GOLD, "windows.psk.d"))
    assert (r.header.version, r.header.sample_ty, len(r)) == (1, "(idx[64][seq: 8], idx[64][seq: 8])", 24)
    x, y = read_leaves(r, oracle_lib, 0, 2)
    assert x.tolist() == [41, 19, 50, 6, 9, 12, 46, 7, 27, 4, 11, 55, 53, 8, 30, 11]
    assert y.tolist() == [19, 50, 6, 9, 12, 46, 7, 27, 4, 11, 55, 53, 8, 30, 11, 54]
    # lm windows: the targets are the inputs shifted by one token
    x, y = read_leaves(r, oracle_lib)
    assert np.array_equal(x.reshape(24, 8)[:, 1:], y.reshape(24, 8)[:, :-1]) and x.max() < 64
    t = pskd.Reader(os.path.join(GOLD, "tokens.psk.d"))
    assert len(t) == 510 and t.layout.sample_bytes() == 16
    tx, ty = read_leaves(t, oracle_lib)
    assert np.array_equal(tx.reshape(-1, 8)[:, 1:], ty.reshape(-1, 8)[:, :-1]) and ty.max() < 64
    for name, ty_text, count in [("pairs.psk.d", "(ℝ[model: 4], ℝ[model: 4])", 128), ("reg.psk.d", "(ℝ[2], ℝ[1])", 256)]:
        r = pskd.Reader(os.path.join(GOLD, name))
        assert (r.header.sample_ty, len(r)) == (ty_text, count)
        vals = read_leaves(r, oracle_lib)
        raw = np.fromfile(os.path.join(GOLD, name), np.uint8)[len(r.header):].view("<f8").reshape(count, -1)
        w = r.layout.leaves()[0].numel
        assert np.array_equal(vals[0].reshape(count, -1), raw[:, :w]) and np.array_equal(vals[1].reshape(count, -1), raw[:, w:])


def test_round_trip_reals_and_indices(tmp_path, oracle_lib):
    ty = "(ℝ[model: 2], idx[10][])"
    layout = Layout.from_type_text(ty)
    p = str(tmp_path / "reals.psk.d")
    assert pskd.write(p, ty, layout, [[[0.5, -1.25], [7]]]) == 1
    r = pskd.Reader(p)
    a, b = read_leaves(r, oracle_lib)
    assert a.tolist() == [0.5, -1.25] and b.tolist() == [7]


def test_version_two_encodings(tmp_path, oracle_lib):
    ty = "(ℝ[a: 3], ℝ[b: 2], idx[5][2], ℝ[])"
    layout = Layout.from_type_text(ty)
    v = [[1.5, -0.25, 3.0], [float(np.float32(0.1)), -2.0], [4, 0], [0.1]]
    encs = [pskd.ENC_BF16, pskd.ENC_F32, pskd.ENC_F64, pskd.ENC_F64]
    p = str(tmp_path / "v2.psk.d")
    pskd.write(p, ty, layout, [v], encs)
    data = open(p, "rb").read()
    assert struct.unpack("<H", data[4:6])[0] == 2, "a narrower leaf: version 2"
    r = pskd.Reader(p)
    assert r.header.encodings == encs
    got = read_leaves(r, oracle_lib)
    assert [g.tolist() for g in got] == v, "every value read back exactly"
    assert len(data) == 4 + 2 + 4 + len(ty.encode()) + 8 + 4 + 4 + 6 + 8 + 2 + 8
    # all f64: version 1, the same bytes as without encodings
    p1, p2 = str(tmp_path / "p1.psk.d"), str(tmp_path / "p2.psk.d")
    pskd.write(p1, ty, layout, [v])
    pskd.write(p2, ty, layout, [v], [pskd.ENC_F64] * 4)
    assert open(p1, "rb").read() == open(p2, "rb").read() and pskd.Reader(p1).header.version == 1
    # 0.1 is no number of f32 or bf16; 0.1f32 none of bf16; an index leaf has no real encoding
    w = [[1.5, 0.1, 3.0], [0.5, 1.0], [1, 2], [1.0]]
    bad = str(tmp_path / "bad.psk.d")
    assert code_of(lambda: pskd.write(bad, ty, layout, [w], [pskd.ENC_F32, pskd.ENC_F64, pskd.ENC_F64, pskd.ENC_F64])) == "E9004"
    assert code_of(lambda: pskd.write(bad, ty, layout, [v], [pskd.ENC_BF16, pskd.ENC_BF16, pskd.ENC_F64, pskd.ENC_F64])) == "E9004"
    assert code_of(lambda: pskd.write(bad, ty, layout, [v], [pskd.ENC_F64, pskd.ENC_F64, pskd.ENC_F32, pskd.ENC_F64])) == "E9005"


def test_version_three_formats(tmp_path, oracle_lib):
    ty = "(ℝ[a: 4], ℝ[b: 3], ℝ[c: 2], idx[5][1])"
    layout = Layout.from_type_text(ty)
    v = [[480.0, -0.375, 2.0 ** -9, -0.0], [65504.0, 1.0 + 2.0 ** -10, -(2.0 ** -24)], [6.0, -0.5], [3]]
    encs = [pskd.Enc.of(pskd.E4M3_SATURATING), pskd.Enc.of(pskd.F16), pskd.Enc.of(pskd.E2M1), pskd.ENC_F64]
    p = str(tmp_path / "v3.psk.d")
    pskd.write(p, ty, layout, [v], encs)
    data = open(p, "rb").read()
    assert struct.unpack("<H", data[4:6])[0] == 3, "a described leaf: version 3"
    r = pskd.Reader(p)
    assert r.header.encodings == encs
    got = read_leaves(r, oracle_lib)
    assert all(math.copysign(1, a) == math.copysign(1, b) and a == b for g, w in zip(got, v) for a, b in zip(g.tolist(), w))
    header = 4 + 2 + 4 + len(ty.encode()) + 8 + 4 + 4 + 3 * 6
    assert len(r.header) == header and len(data) == header + 4 + 6 + 2 + 1
    assert data[header:header + 4] == bytes([0x7F, 0xAC, 0x01, 0x80]), "the E4M3 codes: 480, -1.5*2^-2, 2^-9, -0"
    # a format of its own code is written by it: f32 as a format is version 2
    w = [[1.0] * 4, [0.5] * 3, [2.0] * 2, [0]]
    p2 = str(tmp_path / "own.psk.d")
    pskd.write(p2, ty, layout, [w], [pskd.Enc(3, pskd.F32), pskd.ENC_F64, pskd.ENC_F64, pskd.ENC_F64])
    assert pskd.Reader(p2).header.encodings[0] == pskd.ENC_F32 and pskd.Reader(p2).header.version == 2
    # a value the format does not hold
    bad = [[481.0, 0.0, 0.0, 0.0], [0.0] * 3, [0.0] * 2, [0]]
    assert code_of(lambda: pskd.write(str(tmp_path / "b.psk.d"), ty, layout, [bad], encs)) == "E9004"
    # encoding 3 in a version 2 file; a description that is no format
    v2 = bytearray(data)
    v2[4] = 2
    open(tmp_path / "as2.psk.d", "wb").write(v2)
    assert code_of(lambda: pskd.Reader(str(tmp_path / "as2.psk.d"))) == "E9002"
    odd = bytearray(data)
    odd[4 + 2 + 4 + len(ty.encode()) + 8 + 4 + 1] = 1
    open(tmp_path / "odd.psk.d", "wb").write(odd)
    assert code_of(lambda: pskd.Reader(str(tmp_path / "odd.psk.d"))) == "E9002"


def test_malformed_files(tmp_path):
    (tmp_path / "bad.psk.d").write_bytes(b"NOPE\x01\x00")
    assert code_of(lambda: pskd.Reader(str(tmp_path / "bad.psk.d"))) == "E9002"
    (tmp_path / "short.psk.d").write_bytes(b"PS")
    assert code_of(lambda: pskd.Reader(str(tmp_path / "short.psk.d"))) == "E9002"
    layout = Layout.from_type_text("idx[4][2]")
    ok = str(tmp_path / "ok.psk.d")
    pskd.write(ok, "idx[4][2]", layout, [[[1, 2]], [[3, 0]]])
    (tmp_path / "trunc.psk.d").write_bytes(open(ok, "rb").read()[:-1])
    assert code_of(lambda: pskd.Reader(str(tmp_path / "trunc.psk.d"))) == "E9003"
    assert code_of(lambda: pskd.write(ok, "idx[4][2]", layout, [[[4, 0]]])) == "E9004"
    assert code_of(lambda: pskd.write(ok, "idx[4][2]", layout, [[[0.0, 0.0]]])) == "E9005"
    assert code_of(lambda: pskd.Reader(ok).leaf_bytes(1, 5)) == "E9003"


def test_params_files_need_a_layout(tmp_path, oracle_lib):
    layout = Layout.record([("w", Leaf((2, 1))), ("b", Leaf((1,)))])
    p = str(tmp_path / "theta.psk.d")
    pskd.write(p, "params Linear{2, 1}", layout, [[[0.25, -0.5], [1.0]]])
    r = pskd.Reader(p)
    assert r.layout is None
    assert code_of(lambda: r.leaf_bytes()) == "E9001"
    r = pskd.Reader(p).with_layout(layout)
    assert [x.tolist() for x in read_leaves(r, oracle_lib)] == [[0.25, -0.5], [1.0]]
    # a model of other dimensions: the file is longer than the layout
    small = Layout.record([("w", Leaf((1, 1))), ("b", Leaf((1,)))])
    assert code_of(lambda: pskd.Reader(p).with_layout(small)) == "E9005"

