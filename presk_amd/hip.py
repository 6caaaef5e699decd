"""Python host side of the executor: a ctypes binding of include/presk_hip.h
and `HipExec`, the mirror of the reference's `trait KernelExec`
(crates/presk-kernel/src/host.rs:28-95) over device-resident buffers.

The native library must be built (presk_amd/build.py); nothing here falls
back to a CPU path: a missing library or a device error raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libpresk_hip.so")

EXACT, FAST = 0, 1
OK, ERR, REFUSED, OVERFLOW = 0, -1, -2, -3

STORAGE_BYTES = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3, "i64": 8}

# Every entry point include/presk_hip.h declares.
SYMBOLS = ["presk_hip_init", "presk_hip_last_error", "presk_hip_compile", "presk_hip_run", "presk_hip_run_noalloc",
           "presk_hip_kernel_info",
           "presk_hip_release", "presk_hip_kernel_text", "presk_hip_alloc", "presk_hip_free", "presk_hip_h2d", "presk_hip_d2h", "presk_hip_memset",
           "presk_hip_sync", "presk_hip_stream_create", "presk_hip_stream_destroy", "presk_hip_time",
           "presk_hip_scalar_digest", "presk_hip_batch_create", "presk_hip_batch_add", "presk_hip_batch_graph", "presk_hip_batch_graph_branches",
           "presk_hip_batch_run", "presk_hip_batch_release", "presk_hip_convert", "presk_hip_batch_add_convert",
           "presk_hip_fill_normal", "presk_hip_dropout_mask", "presk_hip_batch_add_dropout",
           "presk_hip_pskd_decode", "presk_hip_pskd_decode_idx", "presk_hip_mfma_probe"]


class HipError(RuntimeError):
    """An executor error, its message starting with the reference's code
    (E10001, E7005, E7007: crates/presk-rt/src/lib.rs:971-981)."""

    def __init__(self, rc: int, message: str):
        super().__init__(message)
        self.rc = rc
        self.code = message.split(":", 1)[0] if message[:1] == "E" else "E10001"


class Info(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_char * 32), ("order", ctypes.c_char * 32), ("guarded", ctypes.c_int32),
                ("n_inputs", ctypes.c_int32), ("split_bound", ctypes.c_int64), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double)]


_lib = None


def lib():
    """The loaded executor library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m presk_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.presk_hip_init.argtypes = [i32]
        L.presk_hip_last_error.restype = ctypes.c_char_p
        L.presk_hip_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i32, i32, ctypes.POINTER(vp)]
        L.presk_hip_run.argtypes = [vp, ctypes.POINTER(vp), i64, i64, vp]
        L.presk_hip_run_noalloc.argtypes = [vp, ctypes.POINTER(vp), i64, i64, vp]
        L.presk_hip_kernel_info.argtypes = [vp, ctypes.POINTER(Info)]
        L.presk_hip_kernel_text.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.presk_hip_kernel_text.restype = i64
        L.presk_hip_release.argtypes = [vp]
        L.presk_hip_release.restype = None
        L.presk_hip_alloc.argtypes = [ctypes.c_size_t, ctypes.POINTER(vp)]
        L.presk_hip_free.argtypes = [vp]
        L.presk_hip_h2d.argtypes = [vp, vp, ctypes.c_size_t, vp]
        L.presk_hip_d2h.argtypes = [vp, vp, ctypes.c_size_t, vp]
        L.presk_hip_memset.argtypes = [vp, i32, ctypes.c_size_t, vp]
        L.presk_hip_sync.argtypes = [vp]
        L.presk_hip_stream_create.argtypes = [ctypes.POINTER(vp)]
        L.presk_hip_stream_destroy.argtypes = [vp]
        L.presk_hip_time.argtypes = [vp, ctypes.POINTER(vp), i64, i64, vp, i32, i32, ctypes.POINTER(ctypes.c_double)]
        L.presk_hip_scalar_digest.argtypes = [i32, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
        L.presk_hip_batch_create.argtypes = [ctypes.POINTER(vp)]
        L.presk_hip_batch_add.argtypes = [vp, vp, ctypes.POINTER(vp), i64, i64]
        L.presk_hip_batch_graph.argtypes = [vp]
        L.presk_hip_batch_graph_branches.argtypes = [vp, i32]
        L.presk_hip_batch_run.argtypes = [vp, vp]
        L.presk_hip_batch_release.argtypes = [vp]
        L.presk_hip_batch_release.restype = None
        L.presk_hip_convert.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_char_p, i64, vp, vp]
        L.presk_hip_fill_normal.argtypes = [vp, ctypes.c_char_p, i64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, vp]
        L.presk_hip_mfma_probe.argtypes = [ctypes.c_char_p, i64, vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        L.presk_hip_pskd_decode.argtypes = [vp, ctypes.c_int, vp, i64, vp, ctypes.c_char_p, vp, vp]
        L.presk_hip_pskd_decode_idx.argtypes = [vp, ctypes.c_uint64, i64, vp, vp]
        L.presk_hip_dropout_mask.argtypes = [vp, ctypes.c_double, ctypes.c_char_p, i64, vp, vp]
        L.presk_hip_batch_add_dropout.argtypes = [vp, vp, ctypes.c_double, ctypes.c_char_p, i64, vp]
        L.presk_hip_batch_add_convert.argtypes = [vp, vp, ctypes.c_char_p, vp, ctypes.c_char_p, i64, vp]
        _lib = L
    return _lib


def check(rc: int):
    if rc != OK:
        raise HipError(rc, lib().presk_hip_last_error().decode())


_initialized = None


def init(device: int = 0):
    """presk_hip_init; device -1 takes PRESK_HIP_DEVICE (device 0 when unset)."""
    global _initialized
    if _initialized != device:
        check(lib().presk_hip_init(device))
        _initialized = device


class DeviceBuffer:
    """A device allocation holding one buffer's storage (codes for f16/e8m15)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().presk_hip_alloc(max(self.nbytes, 1), ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def of(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(lib().presk_hip_h2d(self.ptr, a.ctypes.data, a.nbytes, stream))

    def download(self, dtype, count=None, stream=None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        check(lib().presk_hip_d2h(out.ctypes.data, self.ptr, out.nbytes, stream))
        return out

    def zero(self, stream=None):
        check(lib().presk_hip_memset(self.ptr, 0, self.nbytes, stream))

    def free(self):
        if self.ptr:
            lib().presk_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceView(DeviceBuffer):
    """Bytes [offset, offset + nbytes) of another buffer, which it keeps alive
    and does not free."""

    def __init__(self, parent: DeviceBuffer, offset: int, nbytes: int):
        if offset < 0 or offset + nbytes > parent.nbytes:
            raise ValueError(f"view [{offset}, {offset + nbytes}) outside a buffer of {parent.nbytes} bytes")
        self.parent, self.nbytes = parent, int(nbytes)
        self.ptr = parent.ptr + int(offset)

    def free(self):
        self.ptr = None


class Compiled:
    """A compiled kernel (`KernelFn`)."""

    def __init__(self, text: str, dtype: str, lanes: int = 1, mode: int = FAST):
        h = ctypes.c_void_p()
        rc = lib().presk_hip_compile(text.encode(), dtype.encode(), lanes, mode, ctypes.byref(h))
        check(rc)
        self.handle = h.value
        self.text, self.dtype, self.lanes, self.mode = text, dtype, lanes, mode
        info = Info()
        check(lib().presk_hip_kernel_info(self.handle, ctypes.byref(info)))
        self.kind = info.kind.decode()
        self.order = info.order.decode()
        self.guarded = bool(info.guarded)
        self.n_inputs = info.n_inputs
        # integer (Quant) inputs, `int8/..` or `int4/..` in the header: each
        # has its scales' slot after the output
        head = text.split("->", 1)[0]
        self.n_quant = head.count(": int8/") + head.count(": int4/")
        self.split_bound = info.split_bound
        self.flops = info.flops
        self.bytes = info.bytes

    def read_back(self) -> str:
        """The text as the executor parsed it, printed back."""
        n = lib().presk_hip_kernel_text(self.handle, None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        lib().presk_hip_kernel_text(self.handle, buf, n + 1)
        return buf.value.decode()

    def _table(self, ptrs):
        # the KernelFn table has no length: every slot the kernel reads must
        # be there (inputs, the output, a scales pointer per integer input,
        # the flag when guarded), or the launch would read a pointer past
        # the table's end
        need = self.n_inputs + 1 + self.n_quant + (1 if self.guarded else 0)
        if len(ptrs) < need or any(not p for p in ptrs):
            raise ValueError(f"a KernelFn table of {len(ptrs)} pointers for a kernel of {self.n_inputs} inputs"
                             f"{f' ({self.n_quant} integer, with scales)' if self.n_quant else ''}"
                             f"{' and a flag' if self.guarded else ''}: {need} or more non-null pointers needed")
        return (ctypes.c_void_p * len(ptrs))(*ptrs)

    def run(self, ptrs, lo=0, hi=None, stream=None):
        """One KernelFn call over device pointers [inputs..., output(, flag)]."""
        if hi is None:
            hi = max(self.split_bound, 0)
        check(lib().presk_hip_run(self.handle, self._table(ptrs), lo, hi, stream))

    def time(self, ptrs, warmup=3, reps=20, stream=None, lo=0, hi=None) -> float:
        if hi is None:
            hi = max(self.split_bound, 0)
        ms = ctypes.c_double()
        check(lib().presk_hip_time(self.handle, self._table(ptrs), lo, hi, stream, warmup, reps, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().presk_hip_release(self.handle)
        except Exception:
            pass


def sync(stream=None):
    check(lib().presk_hip_sync(stream))


class HipExec:
    """The `KernelExec` of `--backend hip` (crates/presk-kernel/src/host.rs:28-95):
    runs each kernel of a launch on the device, kernels compiled once per text
    (the native backend's compile-on-first-use, crates/presk-cranelift/src/
    lib.rs:232-430), the overflow flag read after each launch (E7007,
    host.rs:140-177)."""

    def __init__(self, device: int = 0, mode: int = FAST):
        init(device)
        self.mode = mode
        self._cache: dict = {}
        self._flag = DeviceBuffer(4)

    def name(self) -> str:
        return "hip"

    def workers(self) -> int:
        return 1

    def emulates(self) -> bool:
        return False

    def codes(self) -> bool:
        return True

    def compiled(self, text: str, dtype: str, lanes: int = 1) -> Compiled:
        key = (text, dtype, lanes, self.mode)
        c = self._cache.get(key)
        if c is None:
            c = Compiled(text, dtype, lanes, self.mode)
            self._cache[key] = c
        return c

    def run(self, text: str, dtype: str, inputs: list, out: DeviceBuffer, lanes: int = 1, stream=None):
        """`KernelExec::run`: raises HipError E7007 when a narrowing store
        overflowed."""
        c = self.compiled(text, dtype, lanes)
        if len(inputs) != c.n_inputs:
            raise ValueError(f"{len(inputs)} input buffers for a kernel of {c.n_inputs} inputs")
        ptrs = [b.ptr for b in inputs] + [out.ptr]
        if c.guarded:
            self._flag.zero(stream)
            ptrs.append(self._flag.ptr)
        c.run(ptrs, stream=stream)
        if c.guarded:
            if int(self._flag.download(np.uint32, 1, stream)[0]):
                raise HipError(OVERFLOW, f"E7007: the kernel `{text.split(' (')[0][7:]}` stored a finite value past the largest "
                                         f"finite number of {dtype} (an overflow of its storage)")
        return c
