"""Running a presk_amd Program on the CPU through the oracle (test and
cpu-baseline helper): every launch's kernel text executed by oracle/cexec.py
with the interpreter's semantics, buffers held as numpy storage arrays."""
from __future__ import annotations

import concurrent.futures as cf

import numpy as np

from oracle import cexec
from presk_amd import configs


def storage_of(host: dict, p) -> dict:
    """Host f32 values -> storage arrays in each input's declared type."""
    return configs.storage_inputs(p, host)


def compile_all(p, native=False, workers=8):
    texts = {(ln.low.text, ln.low.dtype, ln.low.lanes) for ln in p.launches}
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda t: cexec.compile_kernel(t[0], t[1], t[2], opt="-O3" if native else "-O2", native=native), texts))


_CODES = {"f64": 0, "f32": 1, "bf16": 2, "f16": 4, "e8m15": 5}
_WIDTH = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3}
_NP = {"f64": np.float64, "f32": np.float32, "bf16": np.uint16, "f16": np.uint16, "e8m15": np.uint8}


def _po_convert():
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(cexec.__file__), "liboracle.so"))
    f = lib.po_convert
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    f.restype = ctypes.c_uint32
    return f


def convert(arr: np.ndarray, frm: str, to: str, n: int):
    """The edge conversion of n elements (the oracle's Buf::of(to, to_f64))."""
    src = np.ascontiguousarray(arr).view(np.uint8)
    dst = np.zeros(n * _WIDTH[to], np.uint8)
    flag = _po_convert()(dst.ctypes.data, _CODES[to], src.ctypes.data, _CODES[frm], n)
    return (dst if to == "e8m15" else dst.view(_NP[to])), bool(flag)


def dropout_mask(key: bytes, rate: float, ty: str, n: int) -> np.ndarray:
    """The host's training mask (oracle's po_dropout_mask) in storage form."""
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(cexec.__file__), "liboracle.so"))
    f = lib.po_dropout_mask
    f.argtypes = [ctypes.c_void_p, ctypes.c_double, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p]
    out = np.zeros(max(n, 1) * _WIDTH[ty], np.uint8)
    f((ctypes.c_uint8 * 32)(*key), rate, _CODES[ty], n, out.ctypes.data)
    out = out[: n * _WIDTH[ty]]
    return out if ty == "e8m15" else out.view(_NP[ty])


def run(p, host: dict, threads: int = 1, native: bool = False) -> dict:
    """Executes every launch in order, a kernel reading a buffer of another
    storage type reading it converted at its edge (host.rs:793-829); returns
    the buffers by name (storage)."""
    from presk_amd.configs import _input_specs
    compile_all(p, native=native)
    env = storage_of(host, p)
    types = {}
    # the training dropout masks, from the program's key table (oracle/rng.c)
    for name, slot, rate, ty, count in p.masks:
        env[name] = dropout_mask(p.keys[slot], rate, ty, count)
        types[name] = ty
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, _input_specs(ln.low)):
            if name in env and name not in types:
                types[name] = p.input_types.get(name, ty) if ty != "i64" else ty
            if name in p.quant:
                types[name] = "int"
    # a stacked buffer (Program.stack): its members one after another, read
    # only after every member is written
    stacks = {}
    for m, (parent, first, _, _) in p.bufs.views.items():
        stacks.setdefault(parent, []).append((first, m))
    flag = False
    for ln in p.launches:
        ins = []
        for name, (ty, count) in zip(ln.ins, _input_specs(ln.low)):
            if name not in env and name in stacks:
                members = [m for _, m in sorted(stacks[name])]
                env[name] = np.concatenate([np.asarray(env[m]).ravel() for m in members])
                types[name] = types[members[0]]
            a = env[name]
            if types[name] == "int":
                # integer weights: codes and scales (the KernelFn's slots)
                ins.append((a, env[name + "#scales"]))
                continue
            if types[name] not in ("i64", ln.low.dtype):
                a, f = convert(a, types[name], ln.low.dtype, max(count, 1))
                flag |= f
            ins.append(a)
        out, f = cexec.run(ln.low.text, ln.low.dtype, ins, lanes=ln.low.lanes, threads=threads, native=native)
        env[ln.out] = out
        types[ln.out] = ln.low.dtype if ln.low.out_kind == "real" else "i64"
        flag |= f
    env["__overflow__"] = flag
    return env
