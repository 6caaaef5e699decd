"""Writes tests/golden/digests.json from the reference's own C runtime.

Run in the build container only (it needs /root/reference): `make -C oracle`
first builds oracle/_ref/libpresk_ref.so from the reference's
crates/presk-export-c/c/presk_rt.h and presk_libm.c.  The digests are data:
per function, the order-free digest (oracle/digest.c) of each of its 256
blocks of inputs (every f32 for the f32 functions and conversions, every code
for the widenings, a fixed sample for the narrowings from f64), plus a few
hundred sample input/output pairs per function for readable failures; for
the f64 functions, 16 blocks of their argument sample and their values at the
special arguments of tests/golden/spec.py.

    python tests/golden/make_golden.py [NAME ...]

With names, only those functions are (re)computed and merged into the file.
"""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from tests.golden import spec  # noqa: E402


def main():
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libpresk_ref.so"))
    lib.pd_digest.restype = ctypes.c_uint64
    lib.pd_digest.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64]
    lib.pd_eval.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32), ctypes.c_size_t]
    path = os.path.join(HERE, "digests.json")
    only = sys.argv[1:]
    if only and os.path.exists(path):
        with open(path) as f:
            out = json.load(f)
    else:
        out = {"about": "digests of the reference's presk_rt.h / presk_libm.c (crates/presk-export-c/c), see oracle/digest.c", "functions": {}}
    for name, (fid, domain) in spec.FUNCTIONS.items():
        if only and name not in only:
            continue
        blocks = spec.blocks(domain)
        digs = [format(lib.pd_digest(fid, lo, hi), "016x") for lo, hi in blocks]
        ins = spec.sample_inputs(domain)
        arr_in = (ctypes.c_uint64 * len(ins))(*ins)
        arr_out = (ctypes.c_uint32 * len(ins))()
        assert lib.pd_eval(fid, arr_in, arr_out, len(ins)) == 0
        out["functions"][name] = {"id": fid, "domain": domain, "blocks": digs, "samples": [[i, o] for i, o in zip(ins, arr_out)]}
        print(name, digs[0], flush=True)
    lib.pd_eval_f64.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    out.setdefault("functions_f64", {})
    for name, fid in spec.F64.items():
        if only and name not in only:
            continue
        digs = [format(lib.pd_digest(fid, lo, hi), "016x") for lo, hi in spec.f64_blocks()]
        xs = np.array(spec.f64_specials(), np.float64)
        ys = np.zeros(len(xs), np.uint64)
        assert lib.pd_eval_f64(fid, xs.ctypes.data, ys.ctypes.data, len(xs)) == 0
        out["functions_f64"][name] = {"id": fid, "domain": spec.F64_DOMAIN, "blocks": digs,
                                      "specials": [[format(int(x), "016x"), format(int(y), "016x")]
                                                   for x, y in zip(xs.view(np.uint64), ys)]}
        print(name, digs[0], flush=True)
    with open(path, "w") as f:
        json.dump(out, f, indent=0)


if __name__ == "__main__":
    main()
