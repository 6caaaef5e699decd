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


# ---- attention with RoPE (examples/spec/rope/rope.psk) ------------------------------

ROPE = dict(B=2, T=8, H=2, HD=8, D=16)


def rope_attention(dt, version: int, mode=hip.EXACT):
    """`attention2` (Llama 2's frequencies at base 1e4) or `attention3` (base
    5e5 and Llama 3's scaling, written with clamp) of `Attention.apply` over
    x[batch 2, seq 8, model 16]: the projections as `ein`s, RoPE by slices
    and a concat along `pair`, the scores' `ein`, the scale, the masked
    softmax, the values' `ein` and the output projection summed over (heads,
    hd).  Returns (program, host inputs, {"out": ...})."""
    from presk_amd import llama
    B_, T, H, HD, D = ROPE["B"], ROPE["T"], ROPE["H"], ROPE["HD"], ROPE["D"]
    s = llama.LlamaShape(V=64, D=D, H=H, G=H, FF=16, L=1, B=B_, T=T, base=1e4 if version == 2 else 5e5)
    p = Program(f"rope-attention{version}-{dt}", mode=mode)
    b = Builder(p, dt)
    b.fn = f"attention{version}"
    b.input("x", A(("batch", B_), ("seq", T), ("model", D)))
    for w in ("wq", "wk", "wv"):
        b.input(w, A(("model", D), ("heads", H), ("hd", HD)))
    b.input("wo", A(("heads", H), ("hd", HD), ("model", D)))
    lits = {"two": 2.0, "hdr": float(HD), "base": s.base}
    if version == 3:
        lits.update({"context": 8192.0, "two_pi": 6.283185307179586, "lo": 1.0, "hilo": 3.0, "zero": 0.0, "one": 1.0,
                     "k": 32.0})
    for n in lits:
        b.input(n, A())
    mask = b.causal_mask(T, "mask")
    om = llama._frequencies(b, s)
    if version == 3:
        with b.func("llama3_scaling"):
            # s = clamp((real(context) * w / real(two_pi) - real(lo)) / real(hi - lo), 0, 1)
            sc = b.fused([("mul", [("in", 0), ("in", 1)]), ("div", [("step", 0), ("in", 2)]), ("sub", [("step", 1), ("in", 3)]),
                          ("div", [("step", 2), ("in", 4)]), ("max", [("step", 3), ("in", 5)]), ("min", [("step", 4), ("in", 6)])],
                         ["context", om, "two_pi", "lo", "hilo", "zero", "one"], om, name="s")
            # w * (((1) - s) / real(k) + s)
            om = b.fused([("sub", [("in", 0), ("in", 1)]), ("div", [("step", 0), ("in", 2)]), ("add", [("step", 1), ("in", 1)]),
                          ("mul", [("in", 3), ("step", 2)])], ["one", sc, "k", om], om, name="w3")
    with b.func("angles"):
        rs = b.unary("real", b.positions(T, "ps", axis="seq"), name="rs")
        la, lb = llama.ein_labels(["seq"], ["rot"], ["seq", "rot"])
        phi = b.ein(rs, om, la, lb, ["seq", "rot"], name="phi")
    with b.func("Attention.apply"):
        out_q = ["batch", "heads", "seq", "hd"]
        la, lb = llama.ein_labels(["batch", "seq", "model"], ["model", "heads", "hd"], out_q)
        q = llama._rope(b, s, phi, b.ein("x", "wq", la, lb, out_q, name="qp"), "q")
        k = llama._rope(b, s, phi, b.ein("x", "wk", la, lb, out_q, name="kp"), "k")
        v = b.ein("x", "wv", la, lb, out_q, name="v")
        out_s = ["batch", "heads", "seq", "seq2"]
        la2, lb2 = llama.ein_labels(out_q, out_q, out_s)
        sc = b.ein(q, k, la2, lb2, out_s, name="scores")
        sq = b.unary("sqrt", "hdr", name="sqrt_hd")
        a = b.masked_softmax(b.binary("div", sc, sq, name="scaled"), mask, "seq2", name="probs")
        la3, lb3 = llama.ein_labels(out_s, out_q, out_q)
        o = b.ein(a, v, la3, lb3, out_q, name="o")
        la4, lb4 = llama.ein_labels(out_q, ["heads", "hd", "model"], ["batch", "seq", "model"])
        out = b.ein(o, "wo", la4, lb4, ["batch", "seq", "model"], name="out")
    v_ = inputs()
    host = {"x": v_["rope.x"], "wq": v_["rope.wq"], "wk": v_["rope.wk"], "wv": v_["rope.wv"], "wo": v_["rope.wo"]}
    host.update({n: np.array([x]) for n, x in lits.items()})
    return p, host, {"out": out}


# ---- slices, concat, min/max/clamp and their gradient (examples/spec/concat/concat.psk)


def concat_toy(dt, grad: bool, mode=hip.EXACT):
    """`loss` (and `loss_grad`) of Toy at B 2, T 8: the window's two slices
    (index tensors), the embedding, QKV's weights concatenated along `out`,
    one product, three slices of it, hardtanh (clamp = min(max(x, -1), 1)),
    leaky (max(x, 0.01 x)), min, the head, the mean cross entropy.  The
    gradient is the reference's reverse mode (rules.rs:115-125): for max
    u = heaviside(x0 - x1), for min u = heaviside(x1 - x0), the first operand
    taking ct * u and the second ct * (1 - u) (ties to the second),
    `slice_vjp` for each slice of the product, the concat's cotangent cut
    back by slices, `embed_vjp`.  Returns (program, host, names): "loss",
    and the gradient leaves by path."""
    p = Program(f"concat-{'grad' if grad else 'loss'}-{dt}", mode=mode)
    b = Builder(p, dt)
    B_, T, V, D = 2, 8, 64, 16
    b.input("tok", A(("vocab", V), ("model", D)))
    b.input("head", A(("out", D), ("vocab", V)))
    for w in ("wq", "wk", "wv"):
        b.input(w, A(("model", D), ("out", D)))
    b.input("w", A(("batch", B_), ("seq", T + 1)), "idx")
    for n in ("one", "c001"):
        b.input(n, A())
    with b.func("inputs"):
        ids = b.slice("w", "seq", 0, T, name="ids")
    with b.func("targets"):
        tg = b.slice("w", "seq", 1, T + 1, name="tg")
    with b.func("Toy.apply"):
        x = b.embed("tok", ids, name="x")
    with b.func("QKV.apply"):
        wc = b.concat(b.concat("wq", "wk", "out", name="wqk"), "wv", "out", name="wcat")
        y = b.dot(x, wc, name="y")
        q = b.slice(y, "out", 0, D, name="q")
        k = b.slice(y, "out", D, 2 * D, name="k")
        v = b.slice(y, "out", 2 * D, 3 * D, name="v")
    with b.func("hardtanh"):
        neg1 = b.unary("neg", "one", name="neg1")
        m0 = b.binary("max", q, neg1, name="m0")
        h = b.binary("min", m0, "one", name="h")
    with b.func("leaky"):
        kc = b.binary("mul", k, "c001", name="kc")
        lk = b.binary("max", k, kc, name="lk")
    with b.func("Toy.apply"):
        g = b.fused([("mul", [("in", 0), ("in", 1)]), ("min", [("in", 2), ("in", 3)]), ("add", [("step", 0), ("step", 1)])],
                    [h, lk, v, q], h, name="g")
        logits = b.dot(g, "head", name="logits")
    with b.func("loss"):
        ce = b.cross_entropy(logits, tg, name="ce")
        loss = b.mean_all(ce, name="loss")
    v_ = inputs()
    host = {n: v_["concat." + n] for n in ("tok", "head", "wq", "wk", "wv")}
    host["w"] = v_["concat.w"].astype(np.int64)
    host["one"], host["c001"] = np.array([1.0]), np.array([0.01])
    names = {"loss": loss}
    if not grad:
        return p, host, names
    H1 = [("sub", [("in", 0), ("in", 1)]), ("heaviside", [("step", 0)])]     # u = heaviside(a - b)
    with b.func("loss.vjp"):
        ct_ce = b.mean_vjp("one", ce, None, name="ct_ce")
        ct_lg = b.cross_entropy_vjp(logits, tg, ct_ce, name="ct_logits")
        names["head"] = b.dot_vjp_r(g, ct_lg, name="d.head")
        ct_g = b.dot_vjp_l(ct_lg, "head", name="ct_g")
        ct_h = b.binary("mul", ct_g, lk, name="ct_h")
        ct_lk = b.binary("mul", ct_g, h, name="ct_lk")
        # min(v, q): u = heaviside(q - v) (the second operand less the
        # first); the first operand, v, takes ct * u, q takes ct * (1 - u)
        ct_v = b.fused(H1 + [("mul", [("in", 2), ("step", 1)])], [q, v, ct_g], q, name="ct_v")
        ct_q1 = b.fused(H1 + [("sub", [("in", 3), ("step", 1)]), ("mul", [("in", 2), ("step", 2)])], [q, v, ct_g, "one"], q,
                        name="ct_q_min")
        # min(m0, 1): m0 takes ct * heaviside(1 - m0)
        ct_m0 = b.fused(H1 + [("mul", [("in", 2), ("step", 1)])], ["one", m0, ct_h], m0, name="ct_m0")
        # max(q, -1): q takes ct * heaviside(q - (-1))
        ct_q2 = b.fused(H1 + [("mul", [("in", 2), ("step", 1)])], [q, neg1, ct_m0], q, name="ct_q_ht")
        # max(k, 0.01 k): k takes ct * u, 0.01 k takes ct * (1 - u), whose
        # adjoint is 0.01 times it
        u_k = b.fused(H1, [k, kc], k, name="u_k")
        ct_k1 = b.binary("mul", ct_lk, u_k, name="ct_k_a")
        ct_kc = b.fused([("sub", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("step", 0)])], ["one", u_k, ct_lk], k, name="ct_kc")
        ct_k2 = b.binary("mul", ct_kc, "c001", name="ct_k_b")
        ct_k = b.binary("add", ct_k1, ct_k2, name="ct_k")
        ct_q = b.binary("add", ct_q1, ct_q2, name="ct_q")
        s_q = b.slice_vjp(y, ct_q, "out", 0, D, name="sv_q")
        s_k = b.slice_vjp(y, ct_k, "out", D, 2 * D, name="sv_k")
        s_v = b.slice_vjp(y, ct_v, "out", 2 * D, 3 * D, name="sv_v")
        ct_y = b.binary("add", b.binary("add", s_q, s_k, name="ct_y0"), s_v, name="ct_y")
        d_wc = b.dot_vjp_r(x, ct_y, name="d.wcat")
        ct_x = b.dot_vjp_l(ct_y, wc, name="ct_x")
        # concat's cotangent cut into its operands' slices (rules.rs: Concat)
        d_wqk = b.slice(d_wc, "out", 0, 2 * D, name="d.wqk")
        names["qkv.wq"] = b.slice(d_wqk, "out", 0, D, name="d.wq")
        names["qkv.wk"] = b.slice(d_wqk, "out", D, 2 * D, name="d.wk")
        names["qkv.wv"] = b.slice(d_wc, "out", 2 * D, 3 * D, name="d.wv")
        names["tok"] = b.embed_vjp("tok", ids, ct_x, name="d.tok")
    return p, host, names


# ---- a gradient through a stacked fold (examples/tests/data/stack_grad.psk) ---------


def stack_tower(dt, mode=hip.EXACT):
    """`loss_grad` of Tower (stack{3}(Block), D 3) at B 2: each layer
    x + tanh(x . w + b) * scale (the product with its bias as the epilogue),
    the loss mean(x^2), and the gradient of every layer's w and b by reverse
    mode (tanh's adjoint ct (1 - y^2), the bias's `sum_to`), the layers'
    gradients held in the stacked leaves `d.blocks.w` [3, 3, 3] and
    `d.blocks.b` [3, 3] (their layers are views of them).  Returns
    (program, host, {"blocks.w", "blocks.b"}: each the layers' buffers in
    order)."""
    p = Program(f"stack-grad-{dt}", mode=mode)
    b = Builder(p, dt)
    Lyr, D, B_ = 3, 3, 2
    b.input("x", A(("batch", B_), ("model", D)))
    b.input("scale", A())
    for n in ("one", "two"):
        b.input(n, A())
    for l in range(Lyr):
        b.input(f"b{l}.w", A(D, D))
        b.input(f"b{l}.b", A(D))
    p.stack("blocks.w", [f"b{l}.w" for l in range(Lyr)], dt, D * D)
    p.stack("blocks.b", [f"b{l}.b" for l in range(Lyr)], dt, D)
    p.stack("d.blocks.w", [f"d.b{l}.w" for l in range(Lyr)], dt, D * D)
    p.stack("d.blocks.b", [f"d.b{l}.b" for l in range(Lyr)], dt, D)
    xs, ts = ["x"], []
    for l in range(Lyr):
        with b.func("Block.apply"):
            u = b.dot(xs[-1], f"b{l}.w", f"b{l}.b", name=f"b{l}.u")
            t = b.unary("tanh", u, name=f"b{l}.t")
            xs.append(b.fused([("mul", [("in", 1), ("in", 2)]), ("add", [("in", 0), ("step", 0)])], [xs[-1], t, "scale"], t,
                              name=f"b{l}.out"))
            ts.append(t)
    with b.func("loss"):
        sq = b.unary("pow2", xs[-1], name="sq")
        b.mean_all(sq, name="loss")
    with b.func("loss.vjp"):
        ct_sq = b.mean_vjp("one", sq, None, name="ct_sq")
        ct = b.fused([("mul", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("step", 0)])], ["two", xs[-1], ct_sq], sq, name="ct_x3")
        for l in reversed(range(Lyr)):
            # ct_u = (ct * scale) * (1 - t * t)
            ct_u = b.fused([("mul", [("in", 0), ("in", 1)]), ("mul", [("in", 2), ("in", 2)]), ("sub", [("in", 3), ("step", 1)]),
                            ("mul", [("step", 0), ("step", 2)])], [ct, "scale", ts[l], "one"], ts[l], name=f"ct_u{l}")
            b.sum_to(ct_u, f"b{l}.b", name=f"d.b{l}.b")
            b.dot_vjp_r(xs[l], ct_u, name=f"d.b{l}.w")
            if l > 0:
                ct = b.binary("add", ct, b.dot_vjp_l(ct_u, f"b{l}.w", name=f"ct_xw{l}"), name=f"ct_x{l}")
    v_ = inputs()
    host = {"x": v_["stack.x"], "scale": v_["stack.scale"], "one": np.array([1.0]), "two": np.array([2.0])}
    for l in range(Lyr):
        host[f"b{l}.w"] = v_["stack.w"][l]
        host[f"b{l}.b"] = v_["stack.b"][l]
    return p, host, {"blocks.w": [f"d.b{l}.w" for l in range(Lyr)], "blocks.b": [f"d.b{l}.b" for l in range(Lyr)]}


# ---- next_token (examples/spec/minigpt/serve_minigpt.psk) ------------------------------


def next_token(dt, mode=hip.EXACT):
    """`next_token`'s launches: MiniGPT.apply (its head zeros, as minigpt.psk
    initializes it), the last position (`index seq: -1`) and its division by
    the temperature 0.8.  The draw itself is the host's `sample`
    (crates/presk-kernel/src/host.rs:1659-1688: a host primitive, not a
    kernel), restated by `sample_rows`."""
    p, b, names = gpt.build(MINIGPT, dt, train=False, mode=mode)
    b.input("temp", A())
    with b.func("next_token"):
        last = b.index(names["logits"], "seq", -1, name="last")
        names["scaled"] = b.binary("div", last, "temp", name="scaled")
    host = gpt.host_inputs(MINIGPT)
    host["head"] = np.zeros_like(host["head"])
    host["ids"] = inputs()["next.ctx"].astype(np.int64)
    host["temp"] = np.array([0.8])
    return p, host, names


def sample_rows(logits, us):
    """host.rs:1659-1688: per row, softmax in f64 with musl's exp (exp(x - m)
    over the row's maximum m), then the least index whose running sum of
    e_i / z exceeds the row's uniform draw u; the last index when none does."""
    out = []
    for row, u in zip(np.asarray(logits, np.float64), us):
        m = np.max(row)
        e = [math.exp(x - m) for x in row]
        z = 0.0
        for x in e:
            z += x
        acc, pick = 0.0, len(row) - 1
        for i, x in enumerate(e):
            acc += x / z
            if u < acc:
                pick = i
                break
        out.append(pick)
    return np.array(out)
