"""The measuring backend of `presk solve --measure hip`.

`presk solve` narrows a realization site by site and keeps each narrowing
whose output stays within the error budget.  Each candidate realization is
*measured*: the entry is run under it and its output compared with the
exact reference computed once (crates/presk-driver/src/precision.rs:444-459,
the `measure` closure; its backend chosen at precision.rs:561-569, the
kernel interpreter or the native backend, which computes the interpreter's
bits about twenty times faster).  This module is that backend on the
device: the candidate's program runs in EXACT mode, which computes the
kernel interpreter's bits, so every gap is the interpreter's gap.

The gap is `leaf_gap` (crates/presk-driver/src/gap.rs:57-65): the largest
absolute difference over the output's leaves, +inf where a difference is not
finite.  A candidate the executor cannot run (a realization it refuses,
E7005) or whose run fails (a store past its type's range, E7007) measures
+inf, as `measure` returns f64::INFINITY when the realization cannot be
applied or the call errs.
"""
from __future__ import annotations

import argparse
import json
import math
import sys

import numpy as np

from . import configs, hip
from .realize import Realization


def _or_infinite(x: np.ndarray) -> np.ndarray:
    return np.where(np.isfinite(x), x, np.inf)


def leaf_gap(reference: list, got: list) -> float:
    """gap.rs:57-65 over lists of leaves (f64 arrays): max |a - b|, +inf
    where a difference is not finite (a NaN included)."""
    gap = 0.0
    for a, b in zip(reference, got):
        a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
        if a.size:
            with np.errstate(invalid="ignore", over="ignore"):
                gap = max(gap, float(_or_infinite(np.abs(a - b)).max()))
    return gap


def leaf_max(leaves: list) -> float:
    """gap.rs:44-51: max |x| over the leaves, +inf where x is not finite."""
    out = 0.0
    for a in leaves:
        a = np.asarray(a, np.float64).ravel()
        if a.size:
            out = max(out, float(_or_infinite(np.abs(a)).max()))
    return out


class HipMeasure:
    """measure(realization) -> gap, each candidate run on the device.

    `build(realization)` returns (program, output buffer names) in EXACT
    mode; `host` holds the entry's inputs (host values, f32 or indices);
    `reference` the exact value of each output as f64 arrays.  Compiled
    kernels are shared between candidates (a narrowing changes a few sites;
    the rest compile once)."""

    def __init__(self, build, host: dict, reference: list):
        self.build, self.host = build, host
        self.reference = [np.asarray(r, np.float64) for r in reference]
        self.cache: dict = {}
        self.runs = 0

    def outputs(self, r: Realization) -> list:
        """The candidate's outputs widened to f64 on the device (exactly)."""
        p, names = self.build(r)
        if p.mode != hip.EXACT:
            raise ValueError("a measurement runs the kernel interpreter's bits: build the program in EXACT mode")
        p.compile(self.cache)
        configs.load_inputs(p, self.host)
        p.prepare()
        p.run()
        hip.sync()
        p.check_overflow()
        self.runs += 1
        out = []
        for name in names:
            ty, count = p.bufs.meta[name]
            n = max(count, 1)
            wide = hip.DeviceBuffer(8 * n)
            hip.check(hip.lib().presk_hip_convert(p.bufs.dev[name].ptr, ty.encode(), wide.ptr, b"f64", n, None, None))
            hip.sync()
            out.append(wide.download(np.float64, n))
        return out

    def __call__(self, r: Realization) -> float:
        try:
            got = self.outputs(r)
        except hip.HipError:
            return math.inf
        return leaf_gap(self.reference, got)


def gpt_forward(shape, host: dict):
    """The builder of config 3's entry (the course GPT's loss) for HipMeasure."""
    from . import gpt

    def build(r: Realization):
        p, b, names = gpt.build(shape, r.default, train=False, mode=hip.EXACT, realize=r)
        return p, [names["loss"]]
    return build


def main(argv=None):
    """python -m presk_amd.measure --reference REF.psk.d --realize @A.json [@B.json ...]

    Measures config 3's candidates (the course GPT's loss on the seeded
    batch) against the exact loss held in a .psk.d file (one `ℝ[]` leaf, as
    the reference's interpreter writes it); one JSON line per candidate."""
    from . import gpt, pskd
    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--reference", required=True, help=".psk.d file of the exact output (f64)")
    ap.add_argument("--realize", nargs="+", required=True, help="candidates: a storage type or @FILE each")
    ap.add_argument("--shape", default="course", choices=["course", "tiny"])
    a = ap.parse_args(argv)
    shape = gpt.COURSE if a.shape == "course" else gpt.TINY
    host = gpt.host_inputs(shape)
    r = pskd.Reader(a.reference)
    ref = []
    for i, raw in enumerate(r.leaf_bytes()):
        e = r.header.encoding(i)
        if e.code == 3:
            raise SystemExit("the reference is written in f64, f32 or bf16")
        ref.append(raw.view({0: "<f8", 1: "<f4", 2: "<u2"}[e.code]).astype(np.float64) if e.code != 2 else
                   (raw.view("<u2").astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    m = HipMeasure(gpt_forward(shape, host), host, ref)
    for spec in a.realize:
        gap = m(Realization.parse(spec))
        print(json.dumps({"realization": spec, "gap": gap, "reference_max": leaf_max(ref)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
