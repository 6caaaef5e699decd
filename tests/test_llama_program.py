"""Config 5's program (presk_amd/llama.py) pinned by its mathematics: the
oracle's run of its nests at the TINY shape (f32, every sum in index order)
against an independent float64 Llama forward written with torch -- RMSNorm,
rotary embeddings in Hugging Face's pairing (r with r + HD/2),
grouped-query causal attention, SwiGLU -- on the same weights.  A dropped
term, a transposed operand or a wrong pairing moves the logits far past the
f32 rounding band checked here.  Also: the `ein` relabeling rule on the
program's own cases, and the contraction classes the executor picks."""
import math

import numpy as np
import pytest
import torch

from presk_amd import hip, llama
from tests import cpu_program


def torch_forward(s: llama.LlamaShape, host: dict) -> np.ndarray:
    t = {k: torch.tensor(np.asarray(v), dtype=torch.float64) for k, v in host.items() if k != "ids"}
    ids = torch.tensor(host["ids"])
    B, T, D, G, P, HD = s.B, s.T, s.D, s.G, s.P, s.HD

    def rms(x, g):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + s.eps) * g

    r = torch.arange(HD // 2, dtype=torch.float64)
    w = torch.exp(-2.0 * r / HD * math.log(s.base))
    ang = torch.arange(T, dtype=torch.float64)[:, None] * w[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)

    def rope(x):
        x0, x1 = x[..., : HD // 2], x[..., HD // 2:]
        return torch.cat([x0 * cos - x1 * sin, x1 * cos + x0 * sin], -1)

    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    x = t["tok"][ids]
    for l in range(s.L):
        p = f"b{l}."
        h = rms(x, t[p + "n1.g"])
        q = (h @ t[p + "attn.wq"]).reshape(B, T, G, P, HD).permute(0, 2, 3, 1, 4)
        k = (h @ t[p + "attn.wk"]).reshape(B, T, G, HD).permute(0, 2, 1, 3)
        v = (h @ t[p + "attn.wv"]).reshape(B, T, G, HD).permute(0, 2, 1, 3)
        q, k = rope(q), rope(k)
        sc = (q @ k[:, :, None].transpose(-1, -2).contiguous()) / math.sqrt(HD)
        sc = sc.masked_fill(~mask, float("-inf"))
        a = torch.softmax(sc, -1)
        o = (a @ v[:, :, None]).permute(0, 3, 1, 2, 4).reshape(B, T, D)
        x = x + o @ t[p + "attn.wo"]
        h2 = rms(x, t[p + "n2.g"])
        g = h2 @ t[p + "ff.gate"]
        x = x + (g * torch.sigmoid(g) * (h2 @ t[p + "ff.up"])) @ t[p + "ff.down"]
    return (rms(x, t["norm.g"]) @ t["head"]).numpy()


def test_ein_relabeling():
    assert llama.ein_labels(["batch", "groups", "per", "seq", "hd"], ["batch", "groups", "seq", "hd"],
                            ["batch", "groups", "per", "seq", "seq2"]) == \
        [["batch", "groups", "per", "seq", "hd"], ["batch", "groups", "seq2", "hd"]]
    assert llama.ein_labels(["batch", "groups", "per", "seq", "seq2"], ["batch", "seq", "groups", "hd"],
                            ["batch", "seq", "groups", "per", "hd"]) == \
        [["batch", "groups", "per", "seq", "seq2"], ["batch", "seq2", "groups", "hd"]]
    # nothing dangles: nothing renamed
    assert llama.ein_labels(["batch", "seq", "model"], ["model", "groups", "hd"], ["batch", "groups", "seq", "hd"]) == \
        [["batch", "seq", "model"], ["model", "groups", "hd"]]
    with pytest.raises(ValueError):
        llama.ein_labels(["seq"], ["seq"], ["seq2", "seq3"])


@pytest.mark.parametrize("shape", [llama.TINY, llama.LlamaShape(V=48, D=32, H=4, G=4, FF=40, L=1, B=1, T=6)],
                         ids=["gqa", "mha"])
def test_tiny_llama_logits_against_float64(shape):
    p, b, names = llama.build(shape, "f32", mode=hip.EXACT)
    host = llama.host_inputs(shape)
    env = cpu_program.run(p, host)
    got = env[names["logits"]].astype(np.float64).reshape(shape.B, shape.T, shape.V)
    want = torch_forward(shape, host)
    scale = np.max(np.abs(want))
    err = np.max(np.abs(got - want)) / scale
    assert err < 5e-6, err


def test_contractions_are_mfma_classes():
    p, b, names = llama.build(llama.TINY, "bf16", mode=hip.FAST)
    kinds = {}
    for ln in p.launches:
        c = hip.Compiled(ln.low.text, ln.low.dtype, ln.low.lanes, hip.FAST)
        kinds.setdefault(ln.low.name, c.kind)
    contractions = [n for n in kinds if n == "dot" or n.startswith("ein[batch")]
    assert len(contractions) == 6
    assert all(kinds[n] == "gemm" for n in contractions), kinds
    assert kinds["softmax axis seq2 where"] == "rows"
    assert kinds["mean axis model"] == "rows"
