"""A realization: the storage type of each site of a program, in the
reference's schema (`presk_rt::Realization`, crates/presk-rt/src/lib.rs:370-455):

    {"default": "f32", "order": {"kind": "sequential"},
     "storage":   {"<function>/<let>": "bf16", ...},
     "functions": {"<function>": "f16", ...},
     "params":    {"<parameter path>": "bf16", ...}}

A site's type is its own (`storage`), else its function's (`functions`), else
`default` (`Realization::dtype_at`, lib.rs:446-455).  `params` gives a
parameter's type at rest (rounded once when it is given).  The fields this
executor does not compute -- per-site arithmetic, product and accumulation
formats, affine (`scaled`) activations and integer (`quant`) weights -- are
refused with E7005, as the native backend refuses them.
"""
from __future__ import annotations

import json

STORAGE = ("f64", "f32", "bf16", "f16", "e8m15")


class Realization:
    def __init__(self, default: str, storage=None, functions=None, params=None, order=None):
        for t in [default, *(storage or {}).values(), *(functions or {}).values(), *(params or {}).values()]:
            if t not in STORAGE:
                raise ValueError(f"E7005: the storage type `{t}` is not one the executor computes")
        self.default = default
        self.storage = dict(storage or {})
        self.functions = dict(functions or {})
        self.params = dict(params or {})
        self.order = order or {"kind": "sequential"}

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
        for field in ("arith", "product", "accum", "scaled", "quant"):
            if d.get(field):
                raise ValueError(f"E7005: a realization with `{field}` formats: the kernel interpreter emulates those")
        return cls(d["default"], d.get("storage"), d.get("functions"), d.get("params"), d.get("order"))

    def dtype_at(self, site: str) -> str:
        """The storage type of a site: its own, else its function's, else the default."""
        if site in self.storage:
            return self.storage[site]
        fn = site.split("/", 1)[0]
        return self.functions.get(fn, self.default)

    def param_dtype(self, path: str, host: str = "f32") -> str:
        """A parameter's type at rest: the realization's, else the host's."""
        return self.params.get(path, host)

    def to_json(self) -> dict:
        d = {"default": self.default, "order": self.order}
        if self.storage:
            d["storage"] = self.storage
        if self.functions:
            d["functions"] = self.functions
        if self.params:
            d["params"] = self.params
        return d
