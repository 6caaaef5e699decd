"""The reference's golden entries (tests/golden/run/*.snap, copies of the
reference's tests/run/*.snap: the exact MPFR interpreter's outputs at 256
bits, 12 digits) as programs of the executor's nests, their inputs the ones
`presk run` synthesizes (tests/golden/run/inputs.json, tests/golden/make_run.py).

- `LayerNorm{8}.apply` and `RMSNorm{8}.apply` over x[batch 3, model 8]
  (examples/spec/layernorm/layernorm.psk), gamma ones, beta zeros.
- `mse` and `mse_grad` of `MLP{4, 16}` at B 2 (examples/spec/mlp/mlp.psk):
  Linear (`dot` with its `add` as the epilogue), gelu, Linear, mean of the
  squared error; the gradient of every parameter by reverse mode.
- `MiniGPT.apply` and `loss` at V 64, D 16, H 2, L 2, B 2, T 8: the head
  is initialized to zeros, so these pin the head's products (logits exactly
  0) and the cross entropy of zero logits (ln 64) -- not the blocks.

Each result is compared with the snapshot within the reference's
conformance band |x - x'| <= eps (|x| + a) of the storage type
(crates/presk-kernel/tests/conformance.rs:53-69): f32 (2^-15, 2^-20), bf16
(2^-4, 2^-5)."""
import json
import math
import os
import re

import numpy as np

from presk_amd import gpt, hip
from presk_amd import lower as L
from presk_amd.gpt import Builder
from presk_amd.program import Program

HERE = os.path.dirname(os.path.abspath(__file__))
A = L.ax
BAND = {"f32": (2.0 ** -15, 2.0 ** -20), "bf16": (2.0 ** -4, 2.0 ** -5)}


def inputs() -> dict:
    with open(os.path.join(HERE, "run", "inputs.json")) as f:
        d = json.load(f)
    return {k: np.array([float.fromhex(h) for h in v["f64"]], np.float64).reshape(v["dims"]) for k, v in d.items()}


def snapshot(name: str):
    """The numbers of a snapshot, in order: one array, or {leaf path: array}
    for a record (`params = { l1 = { w = [dims] [...] ... } }`)."""
    with open(os.path.join(HERE, "run", name + ".snap")) as f:
        text = f.read().split("---\n", 2)[2]
    num = r"-?(?:\d+\.?\d*(?:e-?\d+)?|inf|nan)"
    if text.startswith("params = {"):
        out, path = {}, []
        for line in text.splitlines()[1:]:
            s = line.strip()
            if s.endswith("= {"):
                path.append(s.split(" =")[0])
            elif s == "}":
                if path:
                    path.pop()
            elif " = [" in s:
                leaf, rest = s.split(" = ", 1)
                body = rest[rest.index("]") + 1:]
                out[".".join(path + [leaf])] = np.array([float(x) for x in re.findall(num, body)])
        return out
    rest = text.split(" = ", 1)[1]
    if rest.startswith("["):
        rest = rest[rest.index("]") + 1:]
    return np.array([float(x) for x in re.findall(num, rest)])


def within(got, want, dt):
    eps, a = BAND[dt]
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape, (got.shape, want.shape)
    return np.abs(got - want) <= eps * (np.abs(want) + a)


def layernorm(dt, mode=hip.EXACT):
    """`LayerNorm{8}.apply(x, eps = 1e-5)`: mean, (x - mu)^2 (a group), mean,
    (x - mu) / sqrt(var + eps) * gamma + beta (a group)."""
    p = Program(f"layernorm-{dt}", mode=mode)
    X, R, V, E = L.Operand(A(("batch", 3), ("model", 8))), L.Operand(A(("batch", 3))), L.Operand(A(("model", 8))), L.Operand(A())
    p.add(L.reduce_axis("mean", "model", [X], dt), ["x"], "mu")
    p.add(L.fused([("sub", [("in", 0), ("in", 1)]), ("pow2", [("step", 0)])], [X, R], X.axes, dt), ["x", "mu"], "sq")
    p.add(L.reduce_axis("mean", "model", [X], dt), ["sq"], "var")
    p.add(L.fused([("sub", [("in", 0), ("in", 1)]), ("add", [("in", 2), ("in", 3)]), ("sqrt", [("step", 1)]),
                   ("div", [("step", 0), ("step", 2)]), ("mul", [("step", 3), ("in", 4)]), ("add", [("step", 4), ("in", 5)])],
                  [X, R, R, E, V, V], X.axes, dt), ["x", "mu", "var", "eps", "gamma", "beta"], "out")
    host = {"x": inputs()["norm.x"], "eps": np.array([1e-5]), "gamma": np.ones(8), "beta": np.zeros(8)}
    return p, host, "out"


def rmsnorm(dt, mode=hip.EXACT):
    """`RMSNorm{8}.apply(x, eps = 1e-6)`: x * x, mean, {ms + eps, sqrt},
    {x / ., * gamma}."""
    p = Program(f"rmsnorm-{dt}", mode=mode)
    X, R, V, E = L.Operand(A(("batch", 3), ("model", 8))), L.Operand(A(("batch", 3))), L.Operand(A(("model", 8))), L.Operand(A())
    p.add(L.elementwise_binary("mul", [X, X], dt), ["x", "x"], "xx")
    p.add(L.reduce_axis("mean", "model", [X], dt), ["xx"], "ms")
    p.add(L.fused([("add", [("in", 0), ("in", 1)]), ("sqrt", [("step", 0)])], [R, E], R.axes, dt), ["ms", "eps"], "rms")
    p.add(L.fused([("div", [("in", 0), ("in", 1)]), ("mul", [("step", 0), ("in", 2)])], [X, R, V], X.axes, dt),
          ["x", "rms", "gamma"], "out")
    host = {"x": inputs()["norm.x"], "eps": np.array([1e-6]), "gamma": np.ones(8)}
    return p, host, "out"


def mlp(dt, grad: bool, mode=hip.EXACT):
    """`mse` (and `mse_grad`) of MLP{4, 16} at B 2.  Returns (program, host
    inputs, result names: "mse", or the gradient leaves by path)."""
    p = Program(f"mlp-{'grad' if grad else 'mse'}-{dt}", mode=mode)
    b = Builder(p, dt)
    B, D, Hd = 2, 4, 16
    b.input("x", A(("batch", B), ("model", D)))
    b.input("y", A(("batch", B), ("model", D)))
    b.input("l1.w", A(D, Hd))
    b.input("l1.b", A(Hd))
    b.input("l2.w", A(Hd, D))
    b.input("l2.b", A(D))
    b.input("one", A())
    b.input("two", A())
    with b.func("Linear.apply"):
        u = b.dot("x", "l1.w", "l1.b", name="u")
    with b.func("MLP.apply"):
        g = b.unary("gelu", u, name="g")
    with b.func("Linear.apply"):
        yh = b.dot(g, "l2.w", "l2.b", name="yh")
    with b.func("mse"):
        e = b.fused([("sub", [("in", 0), ("in", 1)]), ("pow2", [("step", 0)])], [yh, "y"], yh, name="e")
        loss = b.mean_all(e, name="mse")
    host = {"x": inputs()["mlp.x"], "y": inputs()["mlp.y"], "l1.w": inputs()["mlp.w1"], "l1.b": np.zeros(Hd),
            "l2.w": inputs()["mlp.w2"], "l2.b": np.zeros(D), "one": np.array([1.0]), "two": np.array([2.0])}
    if not grad:
        return p, host, {"mse": loss}
    with b.func("mse.vjp"):
        ct_e = b.mean_vjp("one", e, None, name="ct_e")
        # pow(2)'s adjoint 2 * d * ct, d = yh - y; sub's passes ct on
        ct_y = b.fused([("sub", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("step", 0)]), ("mul", [("step", 1), ("in", 3)])],
                       [yh, "y", "two", ct_e], yh, name="ct_yh")
    with b.func("Linear.apply.vjp"):
        gb2 = b.sum_to(ct_y, "l2.b", name="d.l2.b")
        gw2 = b.dot_vjp_r(g, ct_y, name="d.l2.w")
        ct_g = b.dot_vjp_l(ct_y, "l2.w", name="ct_g")
    with b.func("MLP.apply.vjp"):
        ct_u = b.fused([("gelu_deriv", [("in", 0)]), ("mul", [("in", 1), ("step", 0)])], [u, ct_g], u, name="ct_u")
    with b.func("Linear.apply.vjp"):
        gb1 = b.sum_to(ct_u, "l1.b", name="d.l1.b")
        gw1 = b.dot_vjp_r("x", ct_u, name="d.l1.w")
    return p, host, {"l1.w": gw1, "l1.b": gb1, "l2.w": gw2, "l2.b": gb2}


MINIGPT = gpt.GptShape(V=64, D=16, H=2, L=2, B=2, T=8)


def minigpt(dt, mode=hip.EXACT):
    """The GPT's forward and loss at the MiniGPT snapshots' constants, the
    head zeros (minigpt.psk: `param head ... init = zeros`)."""
    p, b, names = gpt.build(MINIGPT, dt, train=False, mode=mode)
    host = gpt.host_inputs(MINIGPT)
    host["head"] = np.zeros_like(host["head"])
    return p, host, names


LN64 = math.log(64.0)
