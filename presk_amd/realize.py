"""A realization: the storage type of each site of a program, in the
reference's schema (`presk_rt::Realization`, crates/presk-rt/src/lib.rs:370-455):

    {"default": "f32", "order": {"kind": "sequential"},
     "storage":   {"<function>/<let>": "bf16", ...},
     "functions": {"<function>": "f16", ...},
     "params":    {"<parameter path>": "bf16", ...}}

A site's type is its own (`storage`), else its function's (`functions`), else
`default` (`Realization::dtype_at`, lib.rs:446-455).  `params` gives a
parameter's type at rest (rounded once when it is given); `quant` stores a
parameter as integers with per-channel scales (lib.rs:429-433,
crates/presk-rt/src/quant.rs:82-145), both keyed by the parameter's dotted
path in its tree (`blocks.attn.wq.w`, `lnf.γ`), an unknown path refused
with E7001 (lib.rs:697-701).  Per-site arithmetic, product and accumulation
formats and affine (`scaled`) activations are refused with E7005: the
native backend refuses `scaled` (lib.rs:584-589), and the other three are
the kernel interpreter's to emulate.
"""
from __future__ import annotations

import json

from .quant import ABSMAX, POW2, Quant, resolve

STORAGE = ("f64", "f32", "bf16", "f16", "e8m15")


class Realization:
    def __init__(self, default: str, storage=None, functions=None, params=None, order=None, quant=None):
        for t in [default, *(storage or {}).values(), *(functions or {}).values(), *(params or {}).values()]:
            if t not in STORAGE:
                raise ValueError(f"E7005: the storage type `{t}` is not one the executor computes")
        self.default = default
        self.storage = dict(storage or {})
        self.functions = dict(functions or {})
        self.params = dict(params or {})
        self.order = order or {"kind": "sequential"}
        from .lower import order_of
        order_of(self.order)      # refuses an order the schema does not have (E7001)
        self.quant = {}
        for path, q in (quant or {}).items():
            if isinstance(q, Quant):
                self.quant[path] = q
                continue
            bits, scheme = int(q["bits"]), q.get("scheme", ABSMAX)
            if bits not in (8, 4):
                raise ValueError(f"E7001: quantisation to {bits} bits: only 8 and 4 are implemented")
            if scheme not in (ABSMAX, POW2):
                raise ValueError(f"E7001: the quantisation scheme `{scheme}`")
            self.quant[path] = Quant(bits, q["over"], scheme)
        both = sorted(set(self.params) & set(self.quant))
        if both:
            raise ValueError(f"E7001: the parameter `{both[0]}` is both stored in a type of its own and quantised")

    @classmethod
    def uniform(cls, d: str) -> "Realization":
        return cls(d)

    @classmethod
    def parse(cls, spec: str) -> "Realization":
        """`f32`, `bf16`, ... (one type everywhere) or `@PATH` (a file),
        as `Realization::parse` (lib.rs:421-436)."""
        if spec.startswith("@"):
            with open(spec[1:]) as f:
                return cls.of_json(json.load(f))
        return cls.uniform(spec)

    @classmethod
    def of_json(cls, d: dict) -> "Realization":
        for field in ("arith", "product", "accum", "scaled"):
            if d.get(field):
                raise ValueError(f"E7005: a realization with `{field}` formats: the kernel interpreter emulates those")
        return cls(d["default"], d.get("storage"), d.get("functions"), d.get("params"), d.get("order"), d.get("quant"))

    def dtype_at(self, site: str) -> str:
        """The storage type of a site: its own, else its function's, else the default."""
        if site in self.storage:
            return self.storage[site]
        fn = site.split("/", 1)[0]
        return self.functions.get(fn, self.default)

    def param_dtype(self, path: str, host: str = "f32") -> str:
        """A parameter's type at rest: the realization's, else the host's."""
        return self.params.get(path, host)

    def resolve_params(self, leaves: dict, rename: dict):
        """The program buffers the realization's `params` and `quant` paths
        name: `leaves` is {leaf: (axes, the per-layer buffers a stacked leaf
        holds, or None)}, `rename` {dotted path: leaf} where they differ.
        Returns ({buffer: storage type}, {buffer: (Quant, its axis index,
        its axes)}); a stacked leaf's path names each layer's buffer, its
        quantised axis counted on the stacked tensor (a position from the
        end survives the layer axis, quant.rs:20-28) and kept per layer."""
        path_of = {v: k for k, v in rename.items()}
        by_path = {path_of.get(n, n): (n, axes, members) for n, (axes, members) in leaves.items()}
        for path in list(self.params) + list(self.quant):
            if path not in by_path:
                raise ValueError(f"E7001: the realization names the parameter `{path}`, which the program does not have")
        types, quants = {}, {}
        for path, ty in self.params.items():
            n, _, members = by_path[path]
            for m in members or [n]:
                types[m] = ty
        for path, q in self.quant.items():
            n, axes, members = by_path[path]
            over = resolve(q.over, [a.name for a in axes], len(axes))
            if over is None:
                raise ValueError(f"E7001: no axis `{q.over}` to quantise over in `{path}`, a tensor of rank {len(axes)}")
            if members is None:
                quants[n] = (q, over, list(axes))
                continue
            if over == 0:
                raise ValueError(f"E7005: `{path}` quantised over its layer axis: its blocks read dequantised values")
            for m in members:
                quants[m] = (q, over - 1, list(axes[1:]))
        return types, quants

    def to_json(self) -> dict:
        d = {"default": self.default, "order": self.order}
        if self.storage:
            d["storage"] = self.storage
        if self.functions:
            d["functions"] = self.functions
        if self.params:
            d["params"] = self.params
        if self.quant:
            d["quant"] = {p: {"bits": q.bits, "over": q.over, "scheme": q.scheme} for p, q in self.quant.items()}
        return d
