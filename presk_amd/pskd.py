"""`.psk.d` files on the device: the reference's data container
(crates/presk-data/src/lib.rs) -- header, leaf layout, writer -- with every
leaf decoded on the device into the buffer an executor reads it from.

A file is a header then samples of one Presk type, back to back (lib.rs:1-60):

    magic "PSKD" | version u16 | type_len u32, type UTF-8 | count u64
    [v2, v3] leaves u32 | per leaf its encoding u8 (0 f64, 1 f32, 2 bf16,
             3 a float format, followed in v3 by its six parameter bytes)
    samples: the leaves in order; idx[N] as the smallest of u8/u16/u32/u64
             holding N-1; a real leaf in its encoding, little-endian

Reading: the header and layout are host logic (`read_header`, `Layout`); a
leaf's bytes go to device memory as the file holds them and
`presk_hip_pskd_decode` / `presk_hip_pskd_decode_idx` turn them into the
storage type (the exact f64 of each code, stored as Buf::of stores it), in
place of the reader's per-element `Enc::decode` (lib.rs:205-219, 816-843).
Writing (`write`) is the host's `write_encoded` (lib.rs:562-634): a value that
is not a number of its leaf's encoding is refused (E9004).  Error codes are
the reference's: E9001 type not closed, E9002 not a .psk.d file, E9003
truncated, E9004 a value out of its bound, E9005 a type mismatch.
"""
from __future__ import annotations

import ctypes
import math
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import hip

MAGIC = b"PSKD"
VERSION, VERSION_ENCODED, VERSION_FORMATS = 1, 2, 3
DESCRIPTION = 6


class DataError(Exception):
    def __init__(self, code: str, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


# ---- float formats (crates/presk-format/src/lib.rs:101-143) -------------------

SPECIALS = ("ieee", "nan", "none")
OVERFLOWS = ("inf", "nan", "saturate")


@dataclass(frozen=True)
class Format:
    """A binary float format by its parameters: p bits of significand (the
    implicit one included), normal exponents emin..emax, IEEE 754's layout of
    a code (sign, exponent field biased by 1 - emin, p - 1 trailing bits)."""
    p: int
    emin: int
    emax: int
    subnormals: bool = True
    specials: str = "ieee"
    overflow: str = "inf"
    underflow: str = "signed"
    nans: str = "operand"

    @property
    def ebits(self) -> int:
        codes = self.emax - self.emin + 2 + (self.specials == "ieee")
        return (codes & -codes).bit_length() - 1

    @property
    def bits(self) -> int:
        return 1 + self.ebits + self.p - 1

    @property
    def width(self) -> int:
        return (self.bits + 7) // 8

    def check(self) -> "Format":
        """Float::check (lib.rs:220-240)."""
        if not 2 <= self.p <= 53:
            raise ValueError(f"a float format has 2 to 53 bits of significand, not {self.p}")
        if self.emin > self.emax or self.emin < -1022 or self.emax > 1023:
            raise ValueError(f"the exponent range {self.emin}..={self.emax} is not inside f64's")
        codes = self.emax - self.emin + 2 + (self.specials == "ieee")
        if codes & (codes - 1):
            raise ValueError(f"the exponent range {self.emin}..={self.emax} does not fill an exponent field")
        if self.nans == "default" and self.specials == "none":
            raise ValueError("a format with no NaN gives no default NaN")
        ok = self.specials == "ieee" or (self.specials == "nan" and self.overflow in ("nan", "saturate")) or \
            (self.specials == "none" and self.overflow == "saturate")
        if not ok:
            raise ValueError(f"a format with {self.specials} cannot overflow to {self.overflow}")
        return self

    def description(self) -> bytes:
        """The six bytes of a version 3 header (Enc::description, lib.rs:124-140)."""
        flags = int(self.subnormals) | SPECIALS.index(self.specials) << 1 | OVERFLOWS.index(self.overflow) << 3 | \
            int(self.underflow == "positive") << 5 | int(self.nans == "default") << 6
        return struct.pack("<BhhB", self.p, self.emin, self.emax, flags)

    @staticmethod
    def of_description(b: bytes) -> "Format":
        """Enc::of_description (lib.rs:143-166)."""
        p, emin, emax, flags = struct.unpack("<BhhB", bytes(b[:DESCRIPTION]))
        sp, ov = flags >> 1 & 3, flags >> 3 & 3
        if sp > 2:
            raise ValueError(f"special values {sp}")
        if ov > 2:
            raise ValueError(f"overflow {ov}")
        if flags >> 7:
            raise ValueError(f"flags {flags:#04x}")
        return Format(p, emin, emax, bool(flags & 1), SPECIALS[sp], OVERFLOWS[ov],
                      "positive" if flags & 32 else "signed", "default" if flags & 64 else "operand").check()

    def decode(self, code: int) -> float:
        """Float::decode (lib.rs:460-476): the number or special value of a code."""
        t = self.p - 1
        negative = code >> (self.bits - 1) & 1
        top = (1 << self.ebits) - 1
        field, trailing = code >> t & top, code & ((1 << t) - 1)
        if self.specials == "ieee" and field == top:
            v = math.inf if trailing == 0 else math.nan
        elif self.specials == "nan" and field == top and trailing == (1 << t) - 1:
            v = math.nan
        elif field == 0:
            v = math.ldexp(trailing, self.emin - t) if self.subnormals else 0.0
        else:
            v = math.ldexp((1 << t) | trailing, field - (1 - self.emin) - t)
        return -v if negative else v

    def encode(self, x: float) -> int | None:
        """Float::encode (lib.rs:429-458): the code of x when x is a number or
        special value of the format, else None."""
        t = self.p - 1
        neg = math.copysign(1.0, x) < 0
        sign = int(neg) << (self.bits - 1)
        top = (1 << self.ebits) - 1
        if math.isnan(x):
            if self.specials == "none":
                return None
            return sign | top << t | (1 << (t - 1) if self.specials == "ieee" else (1 << t) - 1)
        if math.isinf(x):
            return sign | top << t if self.specials == "ieee" else None
        if x == 0.0:
            return sign
        b = struct.unpack("<Q", struct.pack("<d", abs(x)))[0]
        be, frac = b >> 52, b & ((1 << 52) - 1)
        m, e = (frac, -1074) if be == 0 else (frac | 1 << 52, be - 1075)
        lead = e + m.bit_length() - 1
        if lead > self.emax:
            return None
        if lead < self.emin:
            s = self.emin - t - e
            if s > 0 and m & ((1 << s) - 1):
                return None
            code = sign | (m >> s if s > 0 else m << -s)
        else:
            s = lead - t - e
            if s > 0 and m & ((1 << s) - 1):
                return None
            sig = m >> s if s > 0 else m << -s
            code = sign | (lead + 1 - self.emin) << t | (sig - (1 << t))
        y = self.decode(code)
        return code if y == x and math.copysign(1.0, y) == math.copysign(1.0, x) else None


F64 = Format(53, -1022, 1023)
F32 = Format(24, -126, 127)
BF16 = Format(8, -126, 127)
F16 = Format(11, -14, 15)
E8M15 = Format(16, -126, 127)
E5M2 = Format(3, -14, 15)
E4M3FN = Format(4, -6, 8, True, "nan", "nan")
E4M3_SATURATING = Format(4, -6, 8, True, "none", "saturate", "positive")
E2M1 = Format(2, 0, 2, True, "none", "saturate")


@dataclass(frozen=True)
class Enc:
    """How a real leaf is stored (Enc, lib.rs:80-123): code 0 f64, 1 f32,
    2 bf16, 3 another format by its parameters."""
    code: int
    format: Format

    @staticmethod
    def of(f: Format) -> "Enc":
        return Enc({F64: 0, F32: 1, BF16: 2}.get(f, 3), f)

    @property
    def width(self) -> int:
        return {0: 8, 1: 4, 2: 2}.get(self.code, self.format.width)


ENC_F64, ENC_F32, ENC_BF16 = Enc(0, F64), Enc(1, F32), Enc(2, BF16)


# ---- layout (lib.rs:226-383) ---------------------------------------------------

@dataclass(frozen=True)
class Leaf:
    """`idx[bound][shape]` (bound set) or `ℝ[shape]` (bound None)."""
    shape: tuple
    bound: int | None = None

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def width(self) -> int:
        return idx_width(self.bound) if self.bound is not None else 8


def idx_width(bound: int) -> int:
    """The smallest unsigned integer holding bound - 1 (lib.rs:289-296)."""
    n = max(bound - 1, 0)
    return 1 if n <= 0xFF else 2 if n <= 0xFFFF else 4 if n <= 0xFFFFFFFF else 8


class Layout:
    """A leaf, a tuple of layouts, or a record of named layouts (`params M`)."""

    def __init__(self, leaf: Leaf | None = None, items: list | None = None, names: list | None = None):
        self.leaf, self.items, self.names = leaf, items, names

    def __eq__(self, o):
        return isinstance(o, Layout) and (self.leaf, self.items, self.names) == (o.leaf, o.items, o.names)

    @staticmethod
    def record(fields: list) -> "Layout":
        return Layout(items=[l if isinstance(l, Layout) else Layout(l) for _, l in fields], names=[n for n, _ in fields])

    @staticmethod
    def from_paths(pairs: list) -> "Layout":
        """The record tree of (dotted path, Leaf) pairs given in leaf order
        (`params M`'s leaves: `blocks.attn.wq`, …)."""
        root: dict = {}
        for path, leaf in pairs:
            node = root
            parts = path.split(".")
            for q in parts[:-1]:
                node = node.setdefault(q, {})
            node[parts[-1]] = leaf

        def build(node):
            return Layout.record([(k, build(v) if isinstance(v, dict) else v) for k, v in node.items()])
        return build(root)

    def leaves(self) -> list:
        if self.leaf is not None:
            return [self.leaf]
        return [x for it in self.items for x in it.leaves()]

    def paths(self, prefix: str = "") -> list:
        """Each leaf's dotted path in leaf order: a record's field names, a
        tuple's positions (`params M`'s leaves `blocks.attn.wq.w`, …)."""
        if self.leaf is not None:
            return [prefix]
        out = []
        for i, it in enumerate(self.items):
            key = self.names[i] if self.names is not None else str(i)
            out += it.paths(f"{prefix}.{key}" if prefix else key)
        return out

    def sample_bytes(self, encs: list | None = None) -> int:
        out = 0
        for i, l in enumerate(self.leaves()):
            e = encs[i] if encs else ENC_F64
            out += l.numel * (e.width if l.bound is None else l.width)
        return out

    @staticmethod
    def from_type_text(text: str) -> "Layout":
        """The layout of a closed data type (Layout::from_type_text,
        lib.rs:306-357): ℝ[…] (or Real[…]), idx[N][…], bool[…] (indices below
        2) and tuples of them, every dimension a literal; `params M` needs the
        program (E9001)."""
        p = _TypeParser(text)
        out = p.ty()
        p.end()
        return out


class _TypeParser:
    def __init__(self, text: str):
        self.text, self.i = text, 0

    def fail(self, why: str):
        raise DataError("E9001", f"`{self.text}`: {why}")

    def ws(self):
        while self.i < len(self.text) and self.text[self.i].isspace():
            self.i += 1

    def peek(self, s: str) -> bool:
        self.ws()
        return self.text.startswith(s, self.i)

    def eat(self, s: str):
        if not self.peek(s):
            self.fail(f"`{s}` expected at {self.i}")
        self.i += len(s)

    def word(self) -> str:
        self.ws()
        j = self.i
        while j < len(self.text) and (self.text[j].isalnum() or self.text[j] in "_ℝ."):
            j += 1
        w = self.text[self.i:j]
        self.i = j
        return w

    def nat(self) -> int:
        w = self.word()
        if not w.isdigit():
            self.fail("every dimension of a sample type must be a literal (a `.psk.d` holds concrete tensors)")
        return int(w)

    def axes(self) -> tuple:
        self.eat("[")
        dims = []
        while not self.peek("]"):
            if self.peek("..."):
                self.fail("a sample type cannot have an open prefix `...`")
            save = self.i
            w = self.word()
            if self.peek(":"):
                self.eat(":")
                dims.append(self.nat())
            else:
                self.i = save
                dims.append(self.nat())
            if not self.peek("]"):
                self.eat(",")
        self.eat("]")
        return tuple(dims)

    def ty(self) -> Layout:
        if self.peek("("):
            self.eat("(")
            items = [self.ty()]
            while self.peek(","):
                self.eat(",")
                items.append(self.ty())
            self.eat(")")
            return Layout(items=items)
        w = self.word()
        if w in ("ℝ", "Real"):
            return Layout(Leaf(self.axes()))
        if w == "idx":
            self.eat("[")
            bound = self.nat()
            self.eat("]")
            if bound == 0:
                self.fail("an `idx[0]` has no values")
            return Layout(Leaf(self.axes() if self.peek("[") else (), bound))
        if w == "bool":
            return Layout(Leaf(self.axes() if self.peek("[") else (), 2))
        if w == "params":
            self.fail(f"the layout of `params {self.word()}` needs the program")
        self.fail(f"`{w}` is not a data type (only `ℝ[…]`, `idx[N][…]`, `bool[…]` and tuples of them, with literal dimensions)")

    def end(self):
        self.ws()
        if self.i != len(self.text):
            self.fail(f"unexpected `{self.text[self.i:]}`")


# ---- files (lib.rs:504-780) -------------------------------------------------------

@dataclass
class Header:
    version: int
    sample_ty: str
    count: int
    encodings: list          # per leaf (versions 2, 3); empty in version 1

    def __len__(self) -> int:
        described = sum(1 for e in self.encodings if e.code == 3)
        v2 = 4 + len(self.encodings) + DESCRIPTION * described if self.version >= VERSION_ENCODED else 0
        return 4 + 2 + 4 + len(self.sample_ty.encode()) + 8 + v2

    def encoding(self, i: int) -> Enc:
        return self.encodings[i] if i < len(self.encodings) else ENC_F64


def read_header(path: str) -> tuple:
    """(Header, file length) of a .psk.d file (Reader::open, lib.rs:657-717)."""
    try:
        f = open(path, "rb")
    except OSError as e:
        raise DataError("E9002", f"{path}: {e}")
    with f:
        size = os.fstat(f.fileno()).st_size
        head = f.read(min(size, 1 << 20))
    if len(head) < 4 or head[:4] != MAGIC:
        raise DataError("E9002", f"{path}: not a .psk.d file ({'too short' if len(head) < 4 else 'bad magic'})")

    def take(at, n, what="truncated header"):
        if at + n > len(head):
            raise DataError("E9003", f"{path}: {what}")
        return head[at:at + n]

    (version,) = struct.unpack("<H", take(4, 2))
    if not VERSION <= version <= VERSION_FORMATS:
        raise DataError("E9002", f"{path}: .psk.d version {version}, this tool reads versions {VERSION} to {VERSION_FORMATS}")
    (tlen,) = struct.unpack("<I", take(6, 4))
    try:
        sample_ty = take(10, tlen).decode("utf-8")
    except UnicodeDecodeError:
        raise DataError("E9002", f"{path}: the sample type is not UTF-8")
    at = 10 + tlen
    (count,) = struct.unpack("<Q", take(at, 8))
    at += 8
    encs = []
    if version >= VERSION_ENCODED:
        (n,) = struct.unpack("<I", take(at, 4))
        at += 4
        for i in range(n):
            c = take(at, 1)[0]
            at += 1
            if c == 3 and version == VERSION_FORMATS:
                d = take(at, DESCRIPTION)
                at += DESCRIPTION
                try:
                    f = Format.of_description(d)
                except ValueError as e:
                    raise DataError("E9002", f"{path}: leaf {i}: a format the encoding does not describe ({e})")
                if Enc.of(f).code != 3:
                    raise DataError("E9002", f"{path}: leaf {i}: a format described by its parameters, which has its own code")
                encs.append(Enc(3, f))
            elif c in (0, 1, 2):
                encs.append((ENC_F64, ENC_F32, ENC_BF16)[c])
            else:
                raise DataError("E9002", f"{path}: leaf {i}: unknown encoding {c}")
    return Header(version, sample_ty, count, encs), size


class Reader:
    """A .psk.d file opened for the device: header, layout, and each leaf's
    bytes decoded into device buffers."""

    def __init__(self, path: str, layout: Layout | None = None):
        self.path = path
        self.header, self.file_len = read_header(path)
        self.data_start = len(self.header)
        if layout is None:
            try:
                layout = Layout.from_type_text(self.header.sample_ty)
            except DataError:
                layout = None
        self.layout = None
        if layout is not None:
            self._set(layout, exact=self.header.sample_ty.startswith("params "))

    def with_layout(self, layout: Layout) -> "Reader":
        """Reader::with_layout (lib.rs:730-746): a `params M` file must be
        exactly the size the program's layout implies."""
        self._set(layout, exact=True)
        return self

    def _set(self, layout: Layout, exact: bool):
        leaves = layout.leaves()
        if self.header.version >= VERSION_ENCODED:
            if len(self.header.encodings) != len(leaves):
                raise DataError("E9005", f"{self.path}: {len(self.header.encodings)} encodings for the {len(leaves)} leaves of `{self.header.sample_ty}`")
            for i, l in enumerate(leaves):
                if l.bound is not None and self.header.encodings[i].code != 0:
                    raise DataError("E9005", f"{self.path}: leaf {i} holds indices and has a real encoding")
        size = layout.sample_bytes(self.header.encodings)
        need = self.data_start + self.header.count * size
        have = self.file_len - self.data_start
        if self.file_len < need:
            raise DataError("E9003", f"{self.path}: truncated: {self.header.count} samples of {size} bytes announced, {max(have, 0)} bytes of data present")
        if exact and self.file_len > need:
            raise DataError("E9005", f"{have} bytes of data where {self.header.count} samples of {size} bytes were expected: the file holds a model of other dimensions")
        self.layout = layout

    def _layout(self) -> Layout:
        if self.layout is None:
            Layout.from_type_text(self.header.sample_ty)
        return self.layout

    def __len__(self) -> int:
        return self.header.count

    def leaf_bytes(self, first: int = 0, count: int | None = None) -> list:
        """Per leaf, the raw bytes of samples [first, first + count) as the
        file stores them, each leaf's samples made contiguous."""
        layout = self._layout()
        count = self.header.count - first if count is None else count
        if first < 0 or count < 0 or first + count > self.header.count:
            raise DataError("E9003", f"samples {first}..{first + count} requested, {self.header.count} in the file")
        encs = self.header.encodings
        size = layout.sample_bytes(encs)
        raw = np.fromfile(self.path, dtype=np.uint8, count=count * size, offset=self.data_start + first * size)
        rows = raw.reshape(count, size) if size else raw.reshape(count, 0)
        out, off = [], 0
        for i, l in enumerate(layout.leaves()):
            w = l.width if l.bound is not None else self.header.encoding(i).width
            nb = l.numel * w
            out.append(np.ascontiguousarray(rows[:, off:off + nb]).ravel())
            off += nb
        return out

    def load(self, types: list | str = "f32", first: int = 0, count: int | None = None, stream=None) -> list:
        """Every leaf of samples [first, first + count) in device memory: a
        real leaf in its storage type (`types`, one per leaf or one for all),
        an idx leaf as i64.  Returns (DeviceBuffer, storage type, overflow)
        per leaf, overflow the E7007 guard of an f16/e8m15 store."""
        layout = self._layout()
        leaves = layout.leaves()
        if isinstance(types, str):
            types = [types] * len(leaves)
        out = []
        for i, (leaf, raw) in enumerate(zip(leaves, self.leaf_bytes(first, count))):
            n = raw.size // (leaf.width if leaf.bound is not None else self.header.encoding(i).width)
            src = hip.DeviceBuffer.of(raw) if raw.size else None
            if leaf.bound is not None:
                dst = hip.DeviceBuffer(8 * n)
                hip.check(hip.lib().presk_hip_pskd_decode_idx(src.ptr if src else None, leaf.bound, n, dst.ptr, stream))
                out.append((dst, "i64", False))
            else:
                ty = types[i]
                dst = hip.DeviceBuffer(hip.STORAGE_BYTES[ty] * n)
                flag = hip.DeviceBuffer(4)
                flag.zero(stream)
                e = self.header.encoding(i)
                desc = e.format.description() if e.code == 3 else b""
                dbuf = ctypes.create_string_buffer(desc, DESCRIPTION) if desc else None
                hip.check(hip.lib().presk_hip_pskd_decode(src.ptr if src else None, e.code, dbuf, n, dst.ptr, ty.encode(),
                                                          flag.ptr, stream))
                ovf = bool(flag.download(np.uint32, 1)[0])
                out.append((dst, ty, ovf))
            hip.sync()
        return out


def load_params(p, path: str, layout: Layout, stream=None, rename=None):
    """A `params M` file's leaves decoded straight into a program's declared
    inputs (each in the storage type it was declared in): the buffer of a
    leaf is its dotted path, or `rename[path]` when given (a stacked leaf
    into the buffer its layers are held in)."""
    r = Reader(path).with_layout(layout)
    if r.header.count != 1:
        raise DataError("E9005", f"a parameter file holds one tree, not {r.header.count}")
    names, leaves = layout.paths(), layout.leaves()
    if rename is not None:
        names = [rename.get(n, n) for n in names]
    for i, (name, leaf, raw) in enumerate(zip(names, leaves, r.leaf_bytes())):
        if name not in p.bufs.meta and p.bufs.stacked(name) is not None:
            p.bufs.alloc(name, *p.bufs.stacked(name))
        if name not in p.bufs.meta:
            raise DataError("E9005", f"the program has no input `{name}`")
        ty, n = p.bufs.meta[name]
        if n != leaf.numel:
            raise DataError("E9005", f"`{name}`: {leaf.numel} values in the file, {n} in the program")
        src = hip.DeviceBuffer.of(raw)
        e = r.header.encoding(i)
        desc = ctypes.create_string_buffer(e.format.description(), DESCRIPTION) if e.code == 3 else None
        hip.check(hip.lib().presk_hip_pskd_decode(src.ptr, e.code, desc, n, p.bufs.dev[name].ptr, ty.encode(), None, stream))
        hip.sync()


def write(path: str, sample_ty: str, layout: Layout, samples: list, encs: list | None = None) -> int:
    """write_encoded (lib.rs:571-634): samples as lists of per-leaf flat
    values (ints for idx leaves, floats for real leaves) in leaf order.  The
    file is version 3 when a real leaf is in a described format, 2 when one
    is narrower than f64, else 1."""
    leaves = layout.leaves()
    if encs and len(encs) != len(leaves):
        raise DataError("E9005", f"{len(encs)} encodings for {len(leaves)} leaves")
    enc = [Enc.of(encs[i].format) if encs else ENC_F64 for i in range(len(leaves))]
    for i, l in enumerate(leaves):
        if l.bound is not None and enc[i].code != 0:
            raise DataError("E9005", f"leaf {i} holds indices, which have no real encoding")
    narrow = any(l.bound is None and enc[i].code != 0 for i, l in enumerate(leaves))
    described = any(e.code == 3 for e in enc)
    version = VERSION_FORMATS if described else VERSION_ENCODED if narrow else VERSION
    out = bytearray(MAGIC + struct.pack("<H", version))
    tb = sample_ty.encode()
    out += struct.pack("<I", len(tb)) + tb + struct.pack("<Q", len(samples))
    if narrow:
        out += struct.pack("<I", len(leaves))
        for e in enc:
            out.append(e.code)
            if e.code == 3:
                out += e.format.description()
    for s in samples:
        if len(s) != len(leaves):
            raise DataError("E9005", f"sample has {len(s)} leaves, the type has {len(leaves)}")
        for i, (l, v) in enumerate(zip(leaves, s)):
            v = list(np.asarray(v).ravel())
            if len(v) != l.numel:
                raise DataError("E9005", f"leaf {i}: {len(v)} values, {l.numel} expected")
            if l.bound is not None:
                for x in v:
                    if isinstance(x, (float, np.floating)):
                        raise DataError("E9005", f"leaf {i}: indices expected, reals found")
                    if not 0 <= int(x) < l.bound:
                        raise DataError("E9004", f"leaf {i}: index {x} is not below the bound {l.bound}")
                    out += int(x).to_bytes(8, "little")[:l.width]
            else:
                e = enc[i]
                for x in v:
                    if isinstance(x, (int, np.integer)) and not isinstance(x, bool):
                        raise DataError("E9005", f"leaf {i}: reals expected, indices found")
                    c = e.format.encode(float(x))
                    if c is None:
                        raise DataError("E9004", f"leaf {i}: {x} is not a number of {e.format}")
                    out += c.to_bytes(8, "little")[:e.width]
    with open(path, "wb") as f:
        f.write(out)
    return len(samples)

