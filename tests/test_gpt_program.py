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
