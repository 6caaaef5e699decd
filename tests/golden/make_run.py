"""Writes tests/golden/run/inputs.json: the inputs `presk run` synthesizes for
the reference's golden entries (tests/run/*.snap, written by
crates/presk-interp/tests/run.rs:50-80), drawn as prepare_run draws them
(crates/presk-interp/src/run.rs:74-100, 315-364): the master key
Key::from_seed(0) split into one key per parameter of the entry; a real
tensor N(0, 1) from its key's stream, Box-Muller in f64 (key.rs:53-72) with
the reference's own f64 log and cos; a module's parameters from its
initializer (crates/presk-core/src/lower/init.rs: the key split over its
params and uses in order; xavier_uniform (2u - 1) * sqrt(6 / (fan_in +
fan_out)), crates/presk-interp/src/prims.rs:584-597; zeros; ones).

Run in this container only (it needs the oracle's key library and the
reference's C compiled into oracle/_ref by oracle/Makefile):

    python tests/golden/make_run.py
"""
import ctypes
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


class Keys:
    def __init__(self):
        self.L = ctypes.CDLL(os.path.join(ROOT, "oracle", "liboracle.so"))
        self.R = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libpresk_ref.so"))
        u8 = ctypes.c_uint8 * 32
        self.u8 = u8
        self.L.po_uniform01_at.restype = ctypes.c_double
        self.L.po_uniform01_at.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        self.L.po_key_from_seed.argtypes = [ctypes.c_uint64, ctypes.c_void_p]
        self.L.po_key_split.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        for f in ("presk_log", "presk_cos"):
            getattr(self.R, f).restype = ctypes.c_double
            getattr(self.R, f).argtypes = [ctypes.c_double]

    def from_seed(self, s):
        k = self.u8()
        self.L.po_key_from_seed(s, k)
        return bytes(k)

    def split(self, key, n):
        out = []
        for l in range(n):
            k = self.u8()
            self.L.po_key_split(self.u8(*key), l, k)
            out.append(bytes(k))
        return out

    def uniforms(self, key, n):
        k = self.u8(*key)
        return [self.L.po_uniform01_at(k, e) for e in range(n)]

    def normals(self, key, n):
        k = self.u8(*key)
        e, out = 0, []
        while len(out) < n:
            u1 = self.L.po_uniform01_at(k, e)
            e += 1
            while u1 <= 0.0:
                u1 = self.L.po_uniform01_at(k, e)
                e += 1
            u2 = self.L.po_uniform01_at(k, e)
            e += 1
            out.append(math.sqrt(-2.0 * self.R.presk_log(u1)) * self.R.presk_cos(2.0 * math.pi * u2))
        return out

    def xavier(self, key, fan_in, fan_out):
        bound = math.sqrt(6.0 / (fan_in + fan_out))
        return [(2.0 * u - 1.0) * bound for u in self.uniforms(key, fan_in * fan_out)]


def hexes(v):
    return [float(x).hex() for x in v]


def main():
    K = Keys()
    master = K.from_seed(0)
    out = {}
    # LayerNorm{8}.apply / RMSNorm{8}.apply (layernorm.psk): (θ, x, eps) --
    # θ's initializer draws nothing (ones, zeros)
    keys = K.split(master, 3)
    out["norm.x"] = {"dims": [3, 8], "f64": hexes(K.normals(keys[1], 24))}
    # mse{D = 4}(net, θ : params MLP{4, 16}, x, y) (mlp.psk): the module
    # argument is static, so the keys are θ's, x's and y's
    keys = K.split(master, 3)
    ka, kb = K.split(keys[0], 2)                      # MLP: uses l1, l2
    w1 = K.xavier(K.split(ka, 2)[0], 4, 16)           # Linear: params w, b
    w2 = K.xavier(K.split(kb, 2)[0], 16, 4)
    out["mlp.w1"] = {"dims": [4, 16], "f64": hexes(w1)}
    out["mlp.w2"] = {"dims": [16, 4], "f64": hexes(w2)}
    out["mlp.x"] = {"dims": [2, 4], "f64": hexes(K.normals(keys[1], 8))}
    out["mlp.y"] = {"dims": [2, 4], "f64": hexes(K.normals(keys[2], 8))}
    with open(os.path.join(HERE, "run", "inputs.json"), "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", os.path.join(HERE, "run", "inputs.json"))


if __name__ == "__main__":
    main()
