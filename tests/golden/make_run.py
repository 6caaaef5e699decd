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
    # attention2 / attention3(θ : params Attention, x) (rope.psk): Attention's
    # four params, each normal(std = 0.02) from its key (init.rs: the key split
    # over the module's params in order); x N(0, 1) [batch 2, seq 8, model 16]
    keys = K.split(master, 2)
    kp = K.split(keys[0], 4)
    for name, k, dims in (("wq", kp[0], [16, 2, 8]), ("wk", kp[1], [16, 2, 8]), ("wv", kp[2], [16, 2, 8]),
                          ("wo", kp[3], [2, 8, 16])):
        out["rope." + name] = {"dims": dims, "f64": hexes([v * 0.02 for v in K.normals(k, int(np.prod(dims)))])}
    out["rope.x"] = {"dims": [2, 8, 16], "f64": hexes(K.normals(keys[1], 256))}
    # loss / loss_grad(θ : params Toy, w : Window) (concat.psk): Toy's params
    # tok, head, then its use qkv (QKV's wq, wk, wv), each normal(std = 0.02);
    # the window idx[64][batch 2, seq 9], each index floor(u * 64) of the key's
    # uniform draws (run.rs:325-331)
    keys = K.split(master, 2)
    kt = K.split(keys[0], 3)
    out["concat.tok"] = {"dims": [64, 16], "f64": hexes([v * 0.02 for v in K.normals(kt[0], 64 * 16)])}
    out["concat.head"] = {"dims": [16, 64], "f64": hexes([v * 0.02 for v in K.normals(kt[1], 16 * 64)])}
    kq = K.split(kt[2], 3)
    for name, k in zip(("wq", "wk", "wv"), kq):
        out["concat." + name] = {"dims": [16, 16], "f64": hexes([v * 0.02 for v in K.normals(k, 256)])}
    out["concat.w"] = {"dims": [2, 9], "f64": hexes([float(math.floor(u * 64)) for u in K.uniforms(keys[1], 18)])}
    # loss_grad(θ : params Tower, x, scale) (stack_grad.psk): Tower's one use,
    # stack{3}(Block), its key split over the 3 layers, each Block's w
    # xavier_uniform [3, 3] and b normal(std = 0.5) [3]; x N(0, 1) [batch 2,
    # model 3]; scale a real of no axes, one normal draw
    keys = K.split(master, 3)
    kb = K.split(K.split(keys[0], 1)[0], 3)
    ws, bs = [], []
    for kl in kb:
        k2 = K.split(kl, 2)
        ws += K.xavier(k2[0], 3, 3)
        bs += [v * 0.5 for v in K.normals(k2[1], 3)]
    out["stack.w"] = {"dims": [3, 3, 3], "f64": hexes(ws)}
    out["stack.b"] = {"dims": [3, 3], "f64": hexes(bs)}
    out["stack.x"] = {"dims": [2, 3], "f64": hexes(K.normals(keys[1], 6))}
    out["stack.scale"] = {"dims": [1], "f64": hexes(K.normals(keys[2], 1))}
    # next_token(θ, key, ctx, temperature = 0.8) (serve_minigpt.psk): the
    # key argument is the second of the master's four; sample draws one
    # uniform of it a batch row (host.rs:1659-1688); ctx idx[64][batch 2,
    # seq 8] from the third
    keys = K.split(master, 4)
    out["next.u"] = {"dims": [2], "f64": hexes(K.uniforms(keys[1], 2))}
    out["next.ctx"] = {"dims": [2, 8], "f64": hexes([float(math.floor(u * 64)) for u in K.uniforms(keys[2], 16)])}
    with open(os.path.join(HERE, "run", "inputs.json"), "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", os.path.join(HERE, "run", "inputs.json"))


if __name__ == "__main__":
    main()
