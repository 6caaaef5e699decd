"""Integer weights as the host hands them to the executor: a parameter
quantised per channel (crates/presk-rt/src/quant.rs), and the buffer kind a
kernel input holding it is marked with (`BufKind::of_quant`,
crates/presk-kernel/src/ir.rs:52-79).

A quantised tensor is its integers (int8 one a byte; int4 two a byte, the
even element in the low nibble, two's complement) and one f32 scale per
channel, the channel of a flat index being that index with the `over` axis
removed.  Every load of element e is f32(q_e) * s_c(e), one f32
multiplication (quant.rs:248-252); the executor's KernelFn takes each integer
input's scales in a pointer slot after the output, in input order
(crates/presk-cranelift/src/lib.rs:1619-1624).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

ABSMAX, POW2 = "absmax", "pow2"


@dataclass
class Quant:
    """How a parameter is quantised (quant.rs:82-115): bits 8 or 4, the axis
    the scale is constant along (its position, negative from the end, or
    its name), the scheme."""
    bits: int
    over: object
    scheme: str = ABSMAX

    @property
    def qmax(self) -> int:
        return 2 ** (self.bits - 1) - 1

    def name(self) -> str:
        return f"int{self.bits}" if self.scheme == ABSMAX else f"int{self.bits}/pow2"


@dataclass
class QTensor:
    dims: tuple
    over: int
    quant: Quant
    scales: np.ndarray     # f32, one per index of the axes other than `over`
    data: np.ndarray       # uint8 codes: int8 as bytes, int4 two a byte

    @property
    def numel(self) -> int:
        return int(np.prod(self.dims, dtype=np.int64))

    def split(self):
        return _split(self.dims, self.over)

    def ints(self) -> np.ndarray:
        """The integers, one int8 an element."""
        if self.quant.bits == 8:
            return self.data.view(np.int8)[: self.numel].copy()
        lo = (self.data & 0x0F).astype(np.int8)
        hi = (self.data >> 4).astype(np.int8)
        q = np.empty(2 * self.data.size, np.int8)
        q[0::2], q[1::2] = lo, hi
        q = q[: self.numel]
        return np.where(q >= 8, q - 16, q).astype(np.int8)

    def channels(self) -> np.ndarray:
        _, k, inner = self.split()
        e = np.arange(self.numel, dtype=np.int64)
        return (e // (k * inner)) * inner + e % inner

    def dequantize(self) -> np.ndarray:
        """f32(q) * s, one f32 rounding (quant.rs:177-182)."""
        return (self.ints().astype(np.float32) * self.scales[self.channels()]).astype(np.float32)


def resolve(over, names, rank: int):
    """AxisRef::resolve (quant.rs:44-59): a position (negative from the end)
    or a name that exactly one axis has."""
    if isinstance(over, str):
        hits = [i for i, n in enumerate(names) if n == over]
        return hits[0] if len(hits) == 1 else None
    i = rank + over if over < 0 else over
    return i if 0 <= i < rank else None


def _split(dims, over):
    outer = int(np.prod(dims[:over], dtype=np.int64))
    inner = int(np.prod(dims[over + 1:], dtype=np.int64))
    return outer, int(dims[over]), inner


def _scale_of(m: float, qmax: float, scheme: str) -> np.float32:
    """quant.rs:299-323: absmax m/qmax rounded to f32; pow2 the smallest power
    of two s with m/s <= qmax; 0 for an all-zero channel."""
    if m == 0.0:
        return np.float32(0.0)
    if scheme == ABSMAX:
        return np.float32(m / qmax)
    s = 1.0
    while m / (s / 2.0) <= qmax:
        s /= 2.0
    while m / s > qmax:
        s *= 2.0
    return np.float32(s)


def quantize(w, dims, q: Quant, names=None) -> QTensor:
    """QTensor::quantize (quant.rs:118-145): the weights read in f64, one
    scale a channel from its largest magnitude, each integer x/s rounded to
    nearest even and clamped to +-qmax."""
    if q.bits not in (8, 4):
        raise ValueError(f"E7001: quantisation to {q.bits} bits: only 8 and 4 are implemented")
    dims = tuple(int(d) for d in dims)
    over = resolve(q.over, names or [None] * len(dims), len(dims))
    if over is None:
        raise ValueError(f"E7001: no axis `{q.over}` to quantise over in a tensor of rank {len(dims)}")
    w = np.asarray(w, np.float64).reshape(dims)
    outer, k, inner = _split(dims, over)
    v = w.reshape(outer, k, inner)
    m = np.abs(v).max(axis=1) if k else np.zeros((outer, inner))
    scales = np.array([_scale_of(float(x), q.qmax, q.scheme) for x in m.ravel()], np.float32)
    s = scales.reshape(outer, 1, inner).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(s == 0.0, 0.0, np.round(v / np.where(s == 0.0, 1.0, s)))   # numpy rounds half to even
    ints = np.clip(r, -q.qmax, q.qmax).astype(np.int8).ravel()
    if q.bits == 8:
        data = ints.view(np.uint8).copy()
    else:
        u = (ints.astype(np.int16) & 0x0F).astype(np.uint8)
        if u.size % 2:
            u = np.append(u, np.uint8(0))
        data = (u[0::2] | (u[1::2] << 4)).astype(np.uint8)
    return QTensor(dims, over, q, scales, data)


def of_quant(qt: QTensor, view_dims):
    """BufKind::of_quant (ir.rs:52-79) of a quantised tensor read through a
    view of axes `view_dims`: see `of_quant_dims`."""
    return of_quant_dims(qt.quant.bits, qt.over, qt.dims, view_dims)


def of_quant_dims(bits: int, over: int, stored_dims, view_dims):
    """The (bits, over, span) of a kernel input reading integers stored with
    axes `stored_dims`, scales constant along axis `over`, through a view of
    axes `view_dims` (the elements in their stored order): the run of the
    view's axes that is the stored axis -- the stored axis itself when the
    view keeps it, several when `split` cut it (ir.rs:52-79); None when no
    run of the view's axes is exactly that axis, as after a `merge` of it."""
    _, k, inner = _split(tuple(int(d) for d in stored_dims), over)
    dims = [int(d) for d in view_dims]
    o = over
    if o < len(dims) and dims[o] == k and int(np.prod(dims[o + 1:], dtype=np.int64)) == inner:
        return bits, o, 1
    a, p = len(dims), 1
    while p < inner:
        a -= 1
        if a < 0:
            return None
        p *= dims[a]
    end, kk = a, 1
    while kk < k:
        a -= 1
        if a < 0:
            return None
        kk *= dims[a]
    return (bits, a, end - a) if p == inner and kk == k else None


def kind_text(kind) -> str:
    """The buffer type the kernel text shows (ir.rs:506-507)."""
    bits, over, span = kind
    return f"int{bits}/{over}" if span == 1 else f"int{bits}/{over}..{over + span}"


def mark(text: str, b: int, kind) -> str:
    """The kernel text with input %b marked as integer weights: the host's
    doing (the lowering always emits real loads, ir.rs:20-28)."""
    head, rest = text.split("\n", 1)
    tag = f"%{b} : "
    i = head.index(tag) + len(tag)
    j = head.index("[", i)
    return head[:i] + kind_text(kind) + head[j:] + "\n" + rest
