"""The measured configurations as programs of the reference's nests
(inputs synthetic and seeded).

- `linear` (config 1): `x . w + b`, x f32[batch 4096, 1024] ~ N(0,1),
  w xavier_uniform (crates/presk-kernel/src/host.rs:1641-1656), b ~ N(0, 0.02);
  one `dot+add` (the epilogue plan of lower.rs:846-864).
- `mlp` (config 2): LayerNorm(x[8192, 768]) -> Linear 768->3072 -> GELU ->
  Linear 3072->768 -> residual add, storage bf16 (or f16, e8m15), f32 compute.
  LayerNorm is examples/spec/layernorm/layernorm.psk's: mean, (x-mu)^2, mean,
  (x - mu) / sqrt(var + eps) * gamma + beta, the elementwise chains as fusion
  groups (crates/presk-core/src/fusion.rs:138).
"""
from __future__ import annotations

import math

import numpy as np

from . import lower as L
from .program import Program

A, O = L.ax, L.Operand


def _narrow(x: np.ndarray, t: int, w: int) -> np.ndarray:
    """The code of a float with t fraction and w exponent bits nearest each
    f64, rounded once, ties to even: codes.rs's `narrow`
    (crates/presk-rt/src/codes.rs:29-59) over arrays -- a NaN keeps its sign
    and top payload bits, made quiet; an f64 subnormal is a signed zero; past
    the largest finite number, the infinity."""
    b = np.ascontiguousarray(x, dtype=np.float64).view(np.uint64).ravel()
    one = np.uint64(1)
    sign = (b >> np.uint64(63)) << np.uint64(t + w)
    inf = np.uint64(((1 << w) - 1) << t)
    ab = b & np.uint64((1 << 63) - 1)
    field = (ab >> np.uint64(52)).astype(np.int64)
    m = (ab & np.uint64((1 << 52) - 1)) | np.uint64(1 << 52)
    lead = field - 1023
    bias = (1 << (w - 1)) - 1
    emin = 1 - bias
    shift = 52 - t + np.maximum(emin - lead, 0)
    s = np.minimum(shift, 63).astype(np.uint64)
    q = m >> s
    low = m & ((one << s) - one)
    half = one << (s - one)
    r = q + ((low > half) | ((low == half) & ((q & one) == one))).astype(np.uint64)
    r = np.where(shift > 63, np.uint64(0), r)
    code = np.where(lead >= emin, (np.maximum(lead + bias - 1, 0).astype(np.uint64) << np.uint64(t)) + r, r)
    out = sign | np.minimum(code, inf)
    nan = sign | inf | np.uint64(1 << (t - 1)) | ((ab >> np.uint64(52 - t)) & np.uint64((1 << (t - 1)) - 1))
    out = np.where(ab > np.uint64(0x7FF << 52), nan, out)
    return np.where(field == 0, sign, out)


def encode64(x, ty: str) -> np.ndarray:
    """f64 values -> storage as the host's `Buf::of` makes it
    (crates/presk-rt/src/lib.rs:868-876): f32 and binary16/e8m15 codes rounded
    once from the f64, bf16 through the f32 (`f32_to_bf16(x as f32)`)."""
    x = np.ascontiguousarray(x, dtype=np.float64).ravel()
    if ty == "f64":
        return x.copy()
    if ty in ("f32", "bf16"):
        with np.errstate(over="ignore"):
            return encode(x.astype(np.float32), ty)
    if ty == "f16":
        return _narrow(x, 10, 5).astype(np.uint16)
    if ty == "e8m15":
        c = _narrow(x, 15, 8).astype(np.uint32)
        out = np.empty(c.size * 3, dtype=np.uint8)
        out[0::3], out[1::3], out[2::3] = c & 0xFF, (c >> 8) & 0xFF, (c >> 16) & 0xFF
        return out
    raise ValueError(ty)


def encode(x: np.ndarray, ty: str) -> np.ndarray:
    """f32 values -> storage (rounded once, to nearest even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if ty == "f32":
        return x.ravel()
    if ty == "f64":
        return x.astype(np.float64).ravel()
    b = x.view(np.uint32).astype(np.uint64).ravel()
    if ty == "bf16":
        return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    if ty == "f16":
        return x.astype(np.float16).view(np.uint16).ravel()
    if ty == "e8m15":
        c = ((b + 0x7F + ((b >> 8) & 1)) >> 8).astype(np.uint32)
        out = np.empty(c.size * 3, dtype=np.uint8)
        out[0::3], out[1::3], out[2::3] = c & 0xFF, (c >> 8) & 0xFF, (c >> 16) & 0xFF
        return out
    raise ValueError(ty)


def xavier(rng, n_in, n_out):
    lim = math.sqrt(6.0 / (n_in + n_out))
    return rng.uniform(-lim, lim, size=(n_in, n_out)).astype(np.float32)


def linear(batch=4096, n_in=1024, n_out=1024, dtype="f32", seed=0):
    """Config 1.  Returns (program, host inputs {name: f32 values}, output name, flops)."""
    rng = np.random.default_rng(seed)
    x, w, b = O(A(("batch", batch), n_in)), O(A(n_in, n_out)), O(A(n_out))
    d = L.dot([x, w], dtype)
    p = Program(f"linear-{dtype}")
    p.add(L.dot([x, w, b], dtype, epilogue=(True, d.out_axes)), ["x", "w", "b"], "y")
    host = {"x": rng.standard_normal((batch, n_in)).astype(np.float32), "w": xavier(rng, n_in, n_out),
            "b": (rng.standard_normal(n_out) * 0.02).astype(np.float32)}
    return p, host, "y", 2.0 * batch * n_in * n_out


def mlp(rows=8192, d=768, hidden=3072, dtype="bf16", seed=1):
    """Config 2."""
    rng = np.random.default_rng(seed)
    X = O(A(("batch", rows), ("model", d)))
    R = O(A(("batch", rows)))
    V = O(A(("model", d)))
    E = O(A())
    H = O(A(("batch", rows), hidden))
    p = Program(f"mlp-{dtype}")
    p.add(L.reduce_axis("mean", "model", [X], dtype), ["x"], "mu")
    p.add(L.fused([("sub", [("in", 0), ("in", 1)]), ("pow2", [("step", 0)])], [X, R], X.axes, dtype), ["x", "mu"], "sq")
    p.add(L.reduce_axis("mean", "model", [X], dtype), ["sq"], "var")
    p.add(L.fused([("sub", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("in", 3)]), ("sqrt", [("step", 1)]),
                   ("div", [("step", 0), ("step", 2)]), ("mul", [("step", 3), ("in", 4)]), ("add", [("step", 4), ("in", 5)])],
                  [X, R, R, E, V, V], X.axes, dtype), ["x", "mu", "var", "eps", "gamma", "beta"], "h")
    w1, b1 = O(A(d, hidden)), O(A(hidden))
    d1 = L.dot([X, w1], dtype)
    p.add(L.dot([X, w1, b1], dtype, epilogue=(True, d1.out_axes)), ["h", "w1", "b1"], "u")
    p.add(L.unary("gelu", [H], dtype), ["u"], "g")
    w2, b2 = O(A(hidden, d)), O(A(d))
    d2 = L.dot([H, w2], dtype)
    p.add(L.dot([H, w2, b2], dtype, epilogue=(True, d2.out_axes)), ["g", "w2", "b2"], "y")
    p.add(L.elementwise_binary("add", [X, O(d2.out_axes)], dtype), ["x", "y"], "out")
    host = {"x": rng.standard_normal((rows, d)).astype(np.float32),
            "eps": np.array([1e-5], np.float64),
            "gamma": np.ones(d, np.float32), "beta": np.zeros(d, np.float32),
            "w1": xavier(rng, d, hidden), "b1": (rng.standard_normal(hidden) * 0.02).astype(np.float32),
            "w2": xavier(rng, hidden, d), "b2": (rng.standard_normal(d) * 0.02).astype(np.float32)}
    flops = 2.0 * 2.0 * rows * d * hidden
    return p, host, "out", flops


def storage_inputs(p: Program, host: dict) -> dict:
    """Host values -> each input's storage in its declared type (indices
    int64); an integer weight quantised from its values read in f64
    (QTensor::quantize, crates/presk-rt/src/quant.rs:118-145), its codes
    under its name and its f32 scales under `<name>#scales`."""
    from . import quant as Q
    env = {}
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, _input_specs(ln.low)):
            ty = p.input_types.get(name, ty) if ty != "i64" else ty
            if name in host and name not in env:
                v = host[name]
                if ty == "i64":
                    env[name] = np.ascontiguousarray(v, dtype=np.int64).ravel()
                elif name in p.quant:
                    q, over, axes = p.quant[name]
                    qt = Q.quantize(np.asarray(v, np.float32).astype(np.float64), [a.len for a in axes],
                                    Q.Quant(q.bits, over, q.scheme))
                    env[name], env[name + "#scales"] = qt.data, qt.scales
                elif np.asarray(v).dtype == np.float64:
                    # the host's f64 values (literals, drawn inputs): one Buf::of
                    env[name] = encode64(np.asarray(v).reshape(-1)[:max(count, 1)], ty)
                else:
                    env[name] = encode(np.asarray(v, np.float32).reshape(-1)[:max(count, 1)], ty)
    return env


def load_inputs(p: Program, host: dict):
    """Declares and uploads every host input in the program's storage type."""
    specs = {}
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, _input_specs(ln.low)):
            specs.setdefault(name, (p.input_types.get(name, ty) if ty != "i64" else ty, count))
    for name, arr in storage_inputs(p, host).items():
        if name.endswith("#scales"):
            ty, count = "f32", arr.size
        else:
            ty, count = specs[name]
        p.declare(name, ty, max(count, 1))
        p.bufs.upload(name, arr)


def _input_specs(low: L.Lowered):
    """(storage type, element count) of each input, read off the kernel's header."""
    head = low.text.split("\n", 1)[0]
    if " () -> %" in head:
        return []
    inner = head[head.index(" (%") + 2: head.index(") -> %")]
    specs, depth, cur = [], 0, ""
    for ch in inner:
        depth += ch == "["
        depth -= ch == "]"
        if ch == "," and depth == 0:
            specs.append(cur)
            cur = ""
        else:
            cur += ch
    specs.append(cur)
    out = []
    for s in specs:
        s = s.strip().split(" : ", 1)[1]
        ty, axes = s[: s.index("[")], s[s.index("[") + 1: -1]
        n = 1
        for a in axes.split(", ") if axes else []:
            n *= int(a.split(": ")[-1])
        out.append((ty, n))
    return out
