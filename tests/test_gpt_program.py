"""The course-GPT programs (presk_amd/gpt.py) against an independent model:
the loss and every parameter's gradient of a tiny GPT (V 64, D 16, H 2, L 2,
B 2, T 8; the reference's TINY constants, crates/presk-cranelift/tests/
native.rs) computed by the oracle running the program's nests, against torch
autograd of the same model in float64.  This pins the restated reverse mode
(crates/presk-core/src/ad/rules.rs) by its mathematics."""
import math

import numpy as np
import pytest

from presk_amd import gpt
from tests import cpu_program, fmt

torch = pytest.importorskip("torch")


def torch_model(s, host, masks=None):
    """masks: the program's dropout masks by site (m.emb, b<l>.m.att,
    b<l>.m.res, b<l>.m.ff), applied where 05_gpt.psk drops"""
    M = {k: torch.tensor(np.asarray(v, np.float64)) for k, v in (masks or {}).items()}
    P = {k: torch.tensor(np.asarray(v, np.float64), requires_grad=True) for k, v in host.items()
         if k not in ("ids", "y", "eps", "scale", "two", "one")}
    ids = torch.tensor(host["ids"])
    y = torch.tensor(host["y"])
    eps = float(host["eps"][0])

    def ln(x, g, b):
        mu = x.mean(-1, keepdim=True)
        var = ((x - mu) ** 2).mean(-1, keepdim=True)
        return (x - mu) / torch.sqrt(var + eps) * g + b

    x = P["tok"][ids] + P["pos"][torch.arange(s.T)]
    if M:
        x = x * M["m.emb"].reshape(x.shape)
    mask = torch.tril(torch.ones(s.T, s.T, dtype=torch.bool))
    for l in range(s.L):
        p = f"b{l}."
        h1 = ln(x, P[p + "ln1.g"], P[p + "ln1.b"])
        def heads(t):
            return t.reshape(s.B, s.T, s.H, s.HD).permute(0, 2, 1, 3)
        q = heads(h1 @ P[p + "wq"] + P[p + "wq.b"])
        k = heads(h1 @ P[p + "wk"] + P[p + "wk.b"])
        v = heads(h1 @ P[p + "wv"] + P[p + "wv.b"])
        sc = (q @ k.transpose(-1, -2)) / math.sqrt(s.HD)
        sc = sc.masked_fill(~mask, float("-inf"))
        a = torch.softmax(sc, -1)
        if M:
            a = a * M[p + "m.att"].reshape(a.shape)
        o = (a @ v).permute(0, 2, 1, 3).reshape(s.B, s.T, s.D)
        ao = o @ P[p + "wo"] + P[p + "wo.b"]
        h = x + (ao * M[p + "m.res"].reshape(ao.shape) if M else ao)
        h2 = ln(h, P[p + "ln2.g"], P[p + "ln2.b"])
        u = h2 @ P[p + "up"] + P[p + "up.b"]
        g = 0.5 * u * (1 + torch.erf(u / math.sqrt(2)))
        dn = g @ P[p + "down"] + P[p + "down.b"]
        x = h + (dn * M[p + "m.ff"].reshape(dn.shape) if M else dn)
    xf = ln(x, P["lnf.g"], P["lnf.b"])
    logits = xf @ P["head"]
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, s.V), y.reshape(-1))
    loss.backward()
    return float(loss.detach()), {k: v.grad.numpy() for k, v in P.items()}


@pytest.mark.slow
def test_tiny_gpt_step_matches_autograd():
    s = gpt.TINY
    p, b, names = gpt.build(s, "f32", train=True)
    host = gpt.host_inputs(s)
    env = cpu_program.run(p, host)
    loss = float(fmt.decode(env[names["loss"]], "f32")[0])
    want_loss, want_grads = torch_model(s, host)
    assert abs(loss - want_loss) <= 1e-5 * abs(want_loss), (loss, want_loss)
    assert set(names["grads"]) == set(want_grads)
    # the key bias's gradient is zero in exact arithmetic (a softmax does not
    # see a constant added to a row): errors are measured against each
    # gradient's own scale, floored at a thousandth of the largest
    floor = 1e-3 * max(np.max(np.abs(g)) for g in want_grads.values())
    for name, buf in names["grads"].items():
        got = fmt.decode(env[buf], "f32").astype(np.float64).reshape(want_grads[name].shape)
        want = want_grads[name]
        scale = max(np.max(np.abs(want)), floor)
        err = np.max(np.abs(got - want)) / scale
        assert err < 1e-4, (name, err)


def test_tiny_gpt_step_with_dropout_matches_autograd():
    """the step at the course's dropout 0.2: masks drawn by the oracle from
    the keys 05_gpt.psk's splits give each site, and the same masks applied
    in the torch model -- the loss and every gradient"""
    from presk_amd import keys
    s = gpt.TINY
    p, b, names = gpt.build(s, "f32", train=True, dropout=0.2, step_key=keys.child(keys.from_seed(3), 1))
    host = gpt.host_inputs(s)
    env = cpu_program.run(p, host)
    masks = {name: fmt.decode(env[name], "f32") for name, *_ in p.masks}
    kept = np.mean(np.concatenate(list(masks.values())) > 0)
    assert 0.7 < kept < 0.9 and set(np.unique(np.concatenate(list(masks.values())))) == {0.0, np.float32(1 / 0.8)}
    loss = float(fmt.decode(env[names["loss"]], "f32")[0])
    want_loss, want_grads = torch_model(s, host, masks)
    assert abs(loss - want_loss) <= 1e-5 * abs(want_loss), (loss, want_loss)
    floor = 1e-3 * max(np.max(np.abs(g)) for g in want_grads.values())
    for name, buf in names["grads"].items():
        got = fmt.decode(env[buf], "f32").astype(np.float64).reshape(want_grads[name].shape)
        want = want_grads[name]
        err = np.max(np.abs(got - want)) / max(np.max(np.abs(want)), floor)
        assert err < 1e-4, (name, err)


def adamw_f64(theta, g_all, m, v, t, total, h=gpt.ADAMW):
    """AdamW as optim.rs:1-25 states it (PyTorch's, clip_grad_norm_ included)
    in float64, from given gradients: clip to the global norm c, moments,
    bias corrections 1 - beta^t, decoupled weight decay, cosine schedule
    with warm-up w over `total` steps, t counted from 1."""
    c, b1, b2 = float(h["grad_clip"]), float(h["beta1"]), float(h["beta2"])
    eps, wd, lr0, w = float(h["eps"]), float(h["weight_decay"]), float(h["lr"]), float(h["warmup"])
    norm = math.sqrt(sum(float(np.sum(np.square(g, dtype=np.float64))) for g in g_all.values()))
    factor = min(1.0, c / (norm + 1e-6))
    p = min(1.0, max(0.0, (t - w) / max(total - w, 1.0)))
    lr = lr0 * min(1.0, t / w) * 0.5 * (1 + math.cos(math.pi * p))
    out = {}
    for k, th in theta.items():
        g = g_all[k] * factor
        m2 = b1 * m[k] + (1 - b1) * g
        v2 = b2 * v[k] + (1 - b2) * g * g
        upd = (m2 / (1 - b1 ** t)) / (np.sqrt(v2 / (1 - b2 ** t)) + eps) + wd * th
        out[k] = (th - lr * upd, m2, v2)
    return out, lr, factor


def test_tiny_adamw_step_matches_float64():
    """The program's adamw.step (gpt.adamw) run by the oracle, after a step
    from nonzero moments, against AdamW in float64 from the program's own
    f32 gradients: theta', m' and v' within f32 rounding."""
    s = gpt.TINY
    t, total = 150, 400
    p, b, names = gpt.build(s, "f32", train=True, optimizer=True)
    host = gpt.host_inputs(s)
    host.update(gpt.optimizer_inputs(s, t, total))
    leaves = gpt.opt_leaves(s)
    assert len(leaves) == 21 and sum(1 for _, mem in leaves.values() if mem) == 16
    rng = np.random.default_rng(4)
    for k in leaves:                                   # a later step: moments not at zero
        host["m." + k] = (rng.standard_normal(host["m." + k].size) * 1e-3).astype(np.float32)
        host["v." + k] = (rng.random(host["v." + k].size) * 1e-6).astype(np.float32)
    env = cpu_program.run(p, host)
    dec = lambda name: fmt.decode(env[name], "f32").astype(np.float64)

    def stacked(get, k):
        # a stacked leaf is its layers' values one after another
        mem = leaves[k][1]
        return np.concatenate([get(x) for x in mem]) if mem else get(k)
    grads = {k: stacked(lambda x: dec(names["grads"][x]).ravel(), k) for k in leaves}
    theta = {k: stacked(lambda x: np.asarray(host[x], np.float64).ravel(), k) for k in leaves}
    m = {k: host["m." + k].astype(np.float64) for k in leaves}
    v = {k: host["v." + k].astype(np.float64) for k in leaves}
    want, lr, factor = adamw_f64(theta, grads, m, v, t, total)
    assert 0 < lr < 3e-4 and 0 < factor <= 1
    for k in leaves:
        th2, m2, v2 = (dec(x).ravel() for x in names["adamw"][k])
        wt, wm, wv = want[k]
        assert np.max(np.abs(m2 - wm)) <= 1e-6 * max(np.max(np.abs(wm)), 1e-30), k
        assert np.max(np.abs(v2 - wv)) <= 1e-6 * max(np.max(np.abs(wv)), 1e-30), k
        # theta' = theta - lr * update: the update within f32 rounding of itself, plus theta's own rounding
        assert np.max(np.abs((th2 - theta[k]) - (wt - theta[k]))) <= 1e-5 * lr + 2 ** -23 * np.max(np.abs(theta[k])), k
