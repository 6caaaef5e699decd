"""A sequence of kernel launches over device-resident buffers: the host's
`call_fn` walk (crates/presk-kernel/src/host.rs:887-1039) reduced to what a
fixed entry needs once its nests are known -- each `let` one launch
(`KernelBackend::launch`, host.rs:742-868), every buffer allocated once and
kept in HBM, no copy between launches, the overflow flags read once at the
end of the call.

`Program` holds the launches; `Buffers` the named device allocations.  The
measured configurations (presk_amd/configs.py) are built from it.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip
from . import lower as L

BYTES = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3, "i64": 8, "int8": 1}
INTS = ("int8", "int4")     # integer weights (their f32 scales in `<name>#scales`)


def nbytes(ty: str, count: int) -> int:
    return (count + 1) // 2 if ty == "int4" else count * BYTES[ty]


def numel(axes) -> int:
    n = 1
    for a in axes:
        n *= a.len
    return n


class Buffers:
    """Named device buffers, each with its storage type and element count."""

    def __init__(self):
        self.dev: dict = {}
        self.meta: dict = {}
        # name -> (parent, first element, parent's type, parent's count): a
        # buffer held inside another (a layer's slice of a stacked leaf)
        self.views: dict = {}

    def alloc(self, name: str, ty: str, count: int) -> hip.DeviceBuffer:
        if name in self.dev:
            ty0, c0 = self.meta[name]
            if (ty0, c0) != (ty, count):
                raise ValueError(f"buffer {name} redeclared as {ty}[{count}] (was {ty0}[{c0}])")
            return self.dev[name]
        if name in self.views:
            parent, first, pty, pcount = self.views[name]
            if ty != pty or first + count > pcount:
                raise ValueError(f"buffer {name} ({ty}[{count}]) does not fit {parent} ({pty}[{pcount}]) at {first}")
            whole = self.alloc(parent, pty, pcount)
            if ty == "int4" and first % 2:
                raise ValueError(f"buffer {name}: an int4 slice that starts inside a byte")
            b = hip.DeviceView(whole, nbytes(ty, first), nbytes(ty, count))
            self.dev[name] = b
            self.meta[name] = (ty, count)
            return b
        b = hip.DeviceBuffer(max(nbytes(ty, count), 1))
        self.dev[name] = b
        self.meta[name] = (ty, count)
        return b

    def stacked(self, name: str):
        """(type, count) of `name` when it is the buffer members are held in."""
        for parent, _, ty, count in self.views.values():
            if parent == name:
                return ty, count
        return None

    def upload(self, name: str, storage: np.ndarray):
        self.dev[name].upload(storage)

    def download(self, name: str) -> np.ndarray:
        ty, count = self.meta[name]
        if ty == "e8m15":
            return self.dev[name].download(np.uint8, 3 * count)
        if ty in INTS:
            return self.dev[name].download(np.uint8, nbytes(ty, count))
        dt = {"f64": np.float64, "f32": np.float32, "bf16": np.uint16, "f16": np.uint16, "i64": np.int64}[ty]
        return self.dev[name].download(dt, count)


class Launch:
    def __init__(self, low: L.Lowered, ins: list, out: str, scales=()):
        self.low, self.ins, self.out = low, ins, out
        # the f32 scales of each integer input, in input order: the KernelFn
        # slots after the output (crates/presk-cranelift/src/lib.rs:1619-1624)
        self.scales = list(scales)
        self.compiled: hip.Compiled | None = None
        self.table = None


class Program:
    """Launches in order on one stream; `run` enqueues them all."""

    def __init__(self, name: str, mode: int = hip.FAST):
        self.name = name
        self.mode = mode
        self.launches: list = []
        self.bufs = Buffers()
        self._flag = None
        self._batch = None
        # a host input's storage type when it is not its first reader's (a
        # mixed realization's parameters at rest)
        self.input_types: dict = {}
        # the prepared sequence: ("launch", Launch) and, where a kernel reads a
        # buffer of another storage type, ("convert", src, from, dst, to, n)
        self.steps: list = []
        # training dropout masks (name, key slot, rate, storage type, count),
        # drawn on the device from a table of 32-byte keys (set_keys) before
        # the launches: a mask depends on its key alone
        self.masks: list = []
        self.keys: list = []
        self._keytab = None
        # integer weights: buffer -> (Quant, its quantised axis, its axes),
        # stored as `int8`/`int4` with f32 scales in `<buffer>#scales`
        self.quant: dict = {}

    def add(self, low: L.Lowered, ins: list, out: str, scales=()) -> str:
        """Appends one launch of `low` reading buffers `ins`, writing `out`
        (and `scales`, the scales of its integer inputs)."""
        self.launches.append(Launch(low, list(ins), out, scales))
        return out

    def compile(self, cache: dict | None = None):
        hip.init(0)
        cache = {} if cache is None else cache
        self._flag = hip.DeviceBuffer(4)
        for ln in self.launches:
            key = (ln.low.text, ln.low.dtype, ln.low.lanes, self.mode)
            c = cache.get(key)
            if c is None:
                c = hip.Compiled(ln.low.text, ln.low.dtype, ln.low.lanes, self.mode)
                cache[key] = c
            ln.compiled = c
        return self

    def declare(self, name: str, ty: str, count: int):
        return self.bufs.alloc(name, ty, count)

    def stack(self, parent: str, members: list, ty: str, count: int):
        """Holds buffers `members` (each `count` elements of `ty`) one after
        another in `parent` (`ty`[len(members) * count]): member i is the
        parent's slice i along a new leading axis, with no copy."""
        for i, m in enumerate(members):
            if m in self.bufs.dev or m in self.bufs.views:
                raise ValueError(f"buffer {m} is already allocated or held in a stack")
            self.bufs.views[m] = (parent, i * count, ty, len(members) * count)

    def add_mask(self, name: str, slot: int, rate: float, ty: str, count: int) -> str:
        """A dropout mask `name` (DropoutMask with training on) drawn from key
        `slot` of the key table."""
        self.masks.append((name, slot, float(rate), ty, int(count)))
        return name

    def set_keys(self, keys: list):
        """The key table: one 32-byte key per slot.  Copied to the device by
        prepare(), and at once when the program is already prepared (a
        recorded graph reads the table at each replay)."""
        self.keys = [bytes(k) for k in keys]
        if self._keytab is not None:
            self._upload_keys()

    def _upload_keys(self):
        if not self.keys:
            return
        if self._keytab is None or self._keytab.nbytes < 32 * len(self.keys):
            self._keytab = hip.DeviceBuffer(32 * len(self.keys))
        self._keytab.upload(np.frombuffer(b"".join(self.keys), np.uint8))

    def _key_ptr(self, slot: int) -> int:
        if self._keytab is None or slot >= len(self.keys):
            raise ValueError(f"dropout key slot {slot}: no key table (set_keys)")
        return self._keytab.ptr + 32 * slot

    def prepare(self):
        """Allocates every output and builds each launch's pointer table.  A
        kernel that reads a real buffer of another storage type reads it
        converted at its edge (crates/presk-kernel/src/host.rs:793-829): one
        conversion per buffer and type, before its first such reader -- every
        buffer is written once per call, so later readers see the same
        values."""
        self.steps = []
        converted = {}
        if self.masks:
            self._upload_keys()
        for name, slot, rate, ty, count in self.masks:
            self.bufs.alloc(name, ty, count)
            self.steps.append(("dropout", name, slot, rate, ty, count))
        for ln in self.launches:
            c = ln.compiled
            ty = ln.low.dtype if ln.low.out_kind == "real" else "i64"
            names = []
            for n in ln.ins:
                src_ty, count = self.bufs.meta[n]
                if src_ty not in ("i64", ln.low.dtype) + INTS:
                    key = (n, ln.low.dtype)
                    if key not in converted:
                        dst = f"{n}@{ln.low.dtype}"
                        self.bufs.alloc(dst, ln.low.dtype, count)
                        self.steps.append(("convert", n, src_ty, dst, ln.low.dtype, count))
                        converted[key] = dst
                    n = converted[key]
                names.append(n)
            self.bufs.alloc(ln.out, ty, numel(ln.low.out_axes))
            ptrs = [self.bufs.dev[n].ptr for n in names] + [self.bufs.dev[ln.out].ptr]
            ptrs += [self.bufs.dev[n].ptr for n in ln.scales]
            if c.guarded:
                ptrs.append(self._flag.ptr)
            ln.table = (ctypes.c_void_p * len(ptrs))(*ptrs)
            self.steps.append(("launch", ln))
        self._flag.zero()
        return self

    def _dropout(self, step, stream=None):
        _, name, slot, rate, ty, count = step
        hip.check(hip.lib().presk_hip_dropout_mask(self._key_ptr(slot), rate, ty.encode(), count,
                                                   self.bufs.dev[name].ptr, stream))

    def _convert(self, step, stream=None):
        _, src, frm, dst, to, n = step
        hip.check(hip.lib().presk_hip_convert(self.bufs.dev[src].ptr, frm.encode(), self.bufs.dev[dst].ptr, to.encode(),
                                              n, self._flag.ptr, stream))

    def record(self, graph: bool = True, branches: int = 1):
        """Hands the prepared launch sequence to the executor: `run` then
        issues it from one C call, and with `graph` as one HIP graph launch
        whose independent launches lie on up to `branches` parallel branches."""
        lib = hip.lib()
        self.release_batch()
        b = ctypes.c_void_p()
        hip.check(lib.presk_hip_batch_create(ctypes.byref(b)))
        self._batch = b
        for st in self.steps:
            if st[0] == "dropout":
                _, name, slot, rate, ty, count = st
                hip.check(lib.presk_hip_batch_add_dropout(b, self._key_ptr(slot), rate, ty.encode(), count,
                                                          self.bufs.dev[name].ptr))
                continue
            if st[0] == "convert":
                _, src, frm, dst, to, n = st
                hip.check(lib.presk_hip_batch_add_convert(b, self.bufs.dev[src].ptr, frm.encode(), self.bufs.dev[dst].ptr,
                                                          to.encode(), n, self._flag.ptr))
                continue
            c = st[1].compiled
            hip.check(lib.presk_hip_batch_add(b, c.handle, st[1].table, 0, max(c.split_bound, 0)))
        if graph:
            hip.check(lib.presk_hip_batch_graph_branches(b, branches))
        return self

    def release_batch(self):
        if self._batch is not None:
            hip.lib().presk_hip_batch_release(self._batch)
            self._batch = None

    def __del__(self):
        try:
            self.release_batch()
        except Exception:
            pass

    def run(self, stream=None):
        lib = hip.lib()
        if self._batch is not None:
            hip.check(lib.presk_hip_batch_run(self._batch, stream))
            return
        for st in self.steps:
            if st[0] == "dropout":
                self._dropout(st, stream)
                continue
            if st[0] == "convert":
                self._convert(st, stream)
                continue
            c = st[1].compiled
            rc = lib.presk_hip_run(c.handle, st[1].table, 0, max(c.split_bound, 0), stream)
            if rc:
                hip.check(rc)

    def check_overflow(self):
        """E7007 when any narrowing store of the call overflowed."""
        if int(self._flag.download(np.uint32, 1)[0]):
            raise hip.HipError(hip.OVERFLOW, f"E7007: a store of `{self.name}` overflowed its storage type")

    def kernel_times(self, reps: int = 10, stream=None) -> list:
        """Mean ms of each launch alone (HIP events on the launch stream)."""
        out = []
        for ln in self.launches:
            ms = ctypes.c_double()
            c = ln.compiled
            hip.check(hip.lib().presk_hip_time(c.handle, ln.table, 0, max(c.split_bound, 0), stream, 2, reps, ctypes.byref(ms)))
            out.append((ln, ms.value))
        return out
