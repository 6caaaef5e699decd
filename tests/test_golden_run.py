"""The golden entries on the CPU: the oracle's run of each program
(tests/golden/run_entries.py) against the reference's exact outputs
(tests/golden/run/*.snap) within the storage type's conformance band, and
the inputs' synthesis against the snapshots it feeds -- three independent
snapshots (LayerNorm, RMSNorm, the MLP's loss) agree with float64 models of
the drawn inputs to 1e-11, which pins Key::from_seed / split, the
Box-Muller normals and xavier_uniform's draws (tests/golden/make_run.py)."""
import numpy as np
import pytest
from scipy.special import erf

from tests import cpu_program
from tests.golden import run_entries as R


def test_drawn_inputs_reproduce_the_snapshots_in_f64():
    v = R.inputs()
    x = v["norm.x"]
    mu = x.mean(1, keepdims=True)
    ln = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    rms = x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-6)
    assert np.allclose(ln.ravel(), R.snapshot("layernorm_apply"), rtol=1e-11, atol=1e-12)
    assert np.allclose(rms.ravel(), R.snapshot("rmsnorm_apply"), rtol=1e-11, atol=1e-12)
    u = v["mlp.x"] @ v["mlp.w1"]
    yh = (u * (1 + erf(u / np.sqrt(2))) / 2) @ v["mlp.w2"]
    assert abs(((yh - v["mlp.y"]) ** 2).mean() - R.snapshot("mlp_mse")[0]) < 1e-11


def _oracle(p, host):
    return cpu_program.run(p, host)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("entry", ["layernorm_apply", "rmsnorm_apply"])
def test_norms(entry, dt):
    p, host, out = (R.layernorm if entry == "layernorm_apply" else R.rmsnorm)(dt)
    env = _oracle(p, host)
    from tests import fmt
    got = fmt.decode(env[out], dt)
    assert np.all(R.within(got, R.snapshot(entry), dt))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_mlp_mse_and_grad(dt):
    from tests import fmt
    p, host, names = R.mlp(dt, grad=True)
    env = _oracle(p, host)
    assert np.all(R.within(fmt.decode(env[names["mse"]] if "mse" in names else env["mse"], dt), R.snapshot("mlp_mse"), dt))
    want = R.snapshot("mlp_mse_grad")
    for leaf in ("l1.w", "l1.b", "l2.w", "l2.b"):
        ok = R.within(fmt.decode(env[names[leaf]], dt), want[leaf], dt)
        assert np.all(ok), (leaf, np.flatnonzero(~ok)[:5])


def test_minigpt_zero_head():
    from tests import fmt
    p, host, names = R.minigpt("f32")
    env = _oracle(p, host)
    logits = fmt.decode(env[names["logits"]], "f32")
    assert np.all(logits == 0.0) and R.snapshot("minigpt_forward").size == logits.size
    assert np.all(R.within(env[names["loss"]], R.snapshot("minigpt_loss"), "f32"))


def _rope_f64(v, base, scaled):
    """rope.psk's attention in float64 from the drawn inputs (HF pairing,
    Llama 3's clamp scaling for attention3)."""
    x, wq, wk, wv, wo = v["rope.x"], v["rope.wq"], v["rope.wk"], v["rope.wv"], v["rope.wo"]
    HD, T = 8, 8
    w = np.exp(-2.0 * np.arange(4.0) / HD * np.log(base))
    if scaled:
        s = np.clip((8192.0 * w / 6.283185307179586 - 1.0) / 3.0, 0, 1)
        w = w * ((1 - s) / 32.0 + s)
    phi = np.arange(T)[:, None] * w[None, :]
    c, sn = np.cos(phi), np.sin(phi)

    def rope(t):
        t0, t1 = t[..., :4], t[..., 4:]
        return np.concatenate([t0 * c - t1 * sn, t1 * c + t0 * sn], -1)

    q = rope(np.einsum("bsm,mhd->bhsd", x, wq))
    k = rope(np.einsum("bsm,mhd->bhsd", x, wk))
    vv = np.einsum("bsm,mhd->bhsd", x, wv)
    sc = np.where(np.tril(np.ones((T, T), bool)), np.einsum("bhsd,bhtd->bhst", q, k) / np.sqrt(HD), -np.inf)
    a = np.exp(sc - sc.max(-1, keepdims=True))
    a /= a.sum(-1, keepdims=True)
    return np.einsum("bhsd,hdm->bsm", np.einsum("bhst,bhtd->bhsd", a, vv), wo)


def test_drawn_inputs_reproduce_the_newer_snapshots_in_f64():
    """The attention with RoPE (both frequency rules), the concat toy's loss
    and every gradient leaf, the stacked fold's gradient and next_token's
    two draws, from float64 models (torch autograd for the gradients) of the
    drawn inputs: each within 1e-10 of the exact outputs, which pins the
    key splits of a module's params and uses, normal(std)'s scaling, the
    index draws and the models' mathematics."""
    import torch
    v = R.inputs()
    for name, base, scaled in (("rope_attention2", 1e4, False), ("rope_attention3", 5e5, True)):
        want = R.snapshot(name)
        assert np.allclose(_rope_f64(v, base, scaled).ravel(), want, rtol=1e-10, atol=1e-13), name
    t = lambda k: torch.tensor(v[k], dtype=torch.float64, requires_grad=True)
    tok, head, wq, wk, wv = (t("concat." + n) for n in ("tok", "head", "wq", "wk", "wv"))
    w = torch.tensor(v["concat.w"].astype(np.int64))
    y = tok[w[:, :8]] @ torch.cat([wq, wk, wv], 1)
    q, k, vv = y[..., :16], y[..., 16:32], y[..., 32:]
    g = torch.clamp(q, -1, 1) * torch.maximum(k, k * 0.01) + torch.minimum(vv, q)
    loss = torch.nn.functional.cross_entropy((g @ head).reshape(-1, 64), w[:, 1:].reshape(-1))
    loss.backward()
    assert abs(loss.item() - R.snapshot("concat_loss")[0]) < 1e-10
    want = R.snapshot("concat_loss_grad")
    for leaf, p in (("tok", tok), ("head", head), ("qkv.wq", wq), ("qkv.wk", wk), ("qkv.wv", wv)):
        assert np.max(np.abs(p.grad.numpy().ravel() - want[leaf])) <= 1e-10 * np.max(np.abs(want[leaf])) + 1e-15, leaf
    W, Bb = t("stack.w"), t("stack.b")
    h = torch.tensor(v["stack.x"])
    for l in range(3):
        h = h + torch.tanh(h @ W[l] + Bb[l]) * float(v["stack.scale"][0])
    (h ** 2).mean().backward()
    want = R.snapshot("stack_grad")
    assert np.allclose(W.grad.numpy().ravel(), want["blocks.w"], rtol=1e-10, atol=1e-12)
    assert np.allclose(Bb.grad.numpy().ravel(), want["blocks.b"], rtol=1e-10, atol=1e-12)
    # a zero head gives uniform logits: next_token is the index of each draw
    assert np.array_equal(R.sample_rows(np.zeros((2, 64)), v["next.u"]), R.snapshot("minigpt_next_token"))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_newer_entries_on_the_oracle(dt):
    from tests import fmt
    for ver in (2, 3):
        p, host, names = R.rope_attention(dt, ver)
        env = _oracle(p, host)
        assert np.all(R.within(fmt.decode(env[names["out"]], dt), R.snapshot(f"rope_attention{ver}"), dt)), ver
    p, host, names = R.concat_toy(dt, grad=True)
    env = _oracle(p, host)
    assert np.all(R.within(fmt.decode(env[names["loss"]], dt), R.snapshot("concat_loss"), dt))
    want = R.snapshot("concat_loss_grad")
    for leaf in ("tok", "head", "qkv.wq", "qkv.wk", "qkv.wv"):
        assert np.all(R.within(fmt.decode(env[names[leaf]], dt), want[leaf], dt)), leaf
    p, host, names = R.stack_tower(dt)
    env = _oracle(p, host)
    want = R.snapshot("stack_grad")
    for leaf in ("blocks.w", "blocks.b"):
        got = np.concatenate([fmt.decode(env[n], dt).ravel() for n in names[leaf]])
        assert np.all(R.within(got, want[leaf], dt)), leaf
    p, host, names = R.next_token(dt)
    env = _oracle(p, host)
    scaled = fmt.decode(env[names["scaled"]], dt).reshape(2, 64)
    assert np.array_equal(R.sample_rows(scaled, R.inputs()["next.u"]), R.snapshot("minigpt_next_token"))
