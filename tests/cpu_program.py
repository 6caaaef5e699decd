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


def run(p, host: dict, threads: int = 1, native: bool = False) -> dict:
    """Executes every launch in order; returns the buffers by name (storage)."""
    compile_all(p, native=native)
    env = storage_of(host, p)
    flag = False
    for ln in p.launches:
        out, f = cexec.run(ln.low.text, ln.low.dtype, [env[n] for n in ln.ins], lanes=ln.low.lanes,
                           threads=threads, native=native)
        env[ln.out] = out
        flag |= f
    env["__overflow__"] = flag
    return env
