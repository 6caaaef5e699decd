"""oracle/cexec.py -- TEST INFRASTRUCTURE ONLY (the parity oracle).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything under oracle/.  Never the product path.

The kernel interpreter's native semantics, restated as a C printer: a parsed
kernel (oracle/kernel_text.py) becomes one C11 function that performs exactly
the operations `exec::run_guarded` performs (crates/presk-kernel/src/exec.rs:
619-869 `Env`, 871-896 `run_guarded`/`exec`):

- a kernel of storage type f32, bf16, f16 or e8m15 computes every operation in
  f32, an f64 kernel in f64 (exec.rs:874-885, `Dtype::arith`);
- a load widens exactly (exec.rs:642-665), a store rounds once to the storage
  type (exec.rs:758-782): bf16 by `f32_to_bf16`, f16/e8m15 by the codes'
  narrowing of the value's f64, with the overflow guard's flag set when a
  finite value becomes an infinity (exec.rs:771-778, codes.rs:120-136);
- constants are the f64 literal converted to the arithmetic type
  (exec.rs:113-117 `constant`), an index read as a real is `i as f64` then
  converted (exec.rs:688-689), a real read as an index is `as i64` (Rust's
  saturating cast);
- `+ - * /` are single IEEE operations in the arithmetic type, never fused
  (built with -ffp-contract=off); exp/log/tanh/erf/sin/cos are the
  fdlibm-method functions of oracle/libm.c (f32, or the double ones in an f64
  kernel, exec.rs:115-130); sqrt and abs are IEEE;
- the vector form evaluates every lane of a vector expression, then assigns
  (exec.rs:730-756).

The function has the reference's `KernelFn` ABI, `void f(void *const *bufs,
int64_t lo, int64_t hi)` with the slot order inputs, output, overflow flag
(crates/presk-cranelift/src/lib.rs:38-42, 1609-1629); `[lo, hi)` is the range
of the outermost loop when `Kernel::parallel_outer` (ir.rs:336-373) holds, and
the CPU baseline divides it among OpenMP threads as the native executor divides
it among workers (crates/presk-cranelift/src/lib.rs:1636-1691).
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import re
import subprocess
import tempfile

import numpy as np

from . import kernel_text as kt

HERE = os.path.dirname(os.path.abspath(__file__))
REAL = ("f64", "f32", "bf16", "f16", "e8m15")
BYTES = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3, "i64": 8}
NP_STORAGE = {"f64": np.float64, "f32": np.float32, "bf16": np.uint16, "f16": np.uint16, "e8m15": np.uint8, "i64": np.int64}
WIDTH_RANK = {"f64": 0, "f32": 1, "bf16": 2, "f16": 2, "e8m15": 2}


class Refused(Exception):
    """A kernel the oracle does not restate (quantised weights, non-native
    formats)."""


def _hexlit(x: float) -> str:
    if x != x:
        return "NAN"
    if x == float("inf"):
        return "INFINITY"
    if x == float("-inf"):
        return "(-INFINITY)"
    return float.hex(x)


class _Printer:
    def __init__(self, k: kt.Kernel, dtype: str, lanes: int):
        if k.arith is not None:
            raise Refused(f"non-native formats ({k.arith}) are emulated, not run natively")
        self.k, self.dtype, self.lanes = k, dtype, lanes
        self.A = "double" if dtype == "f64" else "float"
        self.n_in = len(k.inputs)
        self.kinds = []
        # integer weights (BufKind::Quant): buffer -> (scales slot, k, inner)
        self.quant = {}
        for i, b in enumerate(k.bufs):
            q = quant_of(b.ty)
            if q is not None and i < self.n_in:
                bits, over, span = q
                self.kinds.append(f"q{bits}")
                kk, inner = 1, 1
                for d in b.dims[over:over + span]:
                    kk *= d
                for d in b.dims[over + span:]:
                    inner *= d
                self.quant[i] = (self.n_in + 1 + len(self.quant), kk, inner)
            elif b.ty == "i64":
                self.kinds.append("i64")
            elif b.ty in REAL:
                if b.ty != dtype and WIDTH_RANK[b.ty] <= WIDTH_RANK[dtype]:
                    raise Refused(f"buffer %{i} of type {b.ty} in a {dtype} kernel")
                self.kinds.append(b.ty)
            else:
                raise Refused(f"buffer %{i} of type {b.ty}")
        out_kind = self.kinds[-1]
        if out_kind not in ("i64", dtype):
            raise Refused(f"output of type {out_kind} in a {dtype} kernel")
        self.guarded = dtype in ("f16", "e8m15") and out_kind != "i64"
        self.strides = [b.strides() for b in k.bufs]

    # ----- expressions -------------------------------------------------------
    def offset(self, b, ix):
        terms = [f"({self.intx(e)})*{s}" for e, s in zip(ix, self.strides[b])]
        return "(" + (" + ".join(terms) if terms else "0") + ")"

    def load_stored(self, b, off):
        """The buffer's element widened exactly to its own arithmetic type;
        an integer weight's, f32(q) * s with s the scale of its channel
        (exec.rs:653, crates/presk-rt/src/quant.rs:236-252, 295-297)."""
        kind, p = self.kinds[b], f"p{b}"
        if kind in ("q8", "q4"):
            _, kk, inner = self.quant[b]
            q = f"(float){p}[{off}]" if kind == "q8" else f"(float)oc_nibble({p}, {off})"
            return f"({q} * sc{b}[(({off}) / {kk * inner}) * {inner} + ({off}) % {inner}])"
        if kind in ("f32", "f64"):
            return f"{p}[{off}]"
        if kind == "bf16":
            return f"oc_bf16_to_f32({p}[{off}])"
        if kind == "f16":
            return f"oc_f16_to_f32({p}[{off}])"
        if kind == "e8m15":
            return f"oc_e8m15_to_f32(ld24({p}, {off}))"
        raise AssertionError(kind)

    def real(self, e):
        A = self.A
        tag = e[0]
        if tag == "num":
            return f"(({A}){_hexlit(float(e[1]))})"
        if tag == "load":
            b, off = e[1], self.offset(e[1], e[2])
            if self.kinds[b] == "i64":
                return f"(({A})(double)p{b}[{off}])"
            return f"(({A}){self.load_stored(b, off)})"
        if tag == "sv":
            return f"s{e[1]}"
        if tag in ("iv", "si"):
            return f"(({A})(double)({self.intx(e)}))"
        if tag == "bin":
            return f"({self.real(e[2])} {e[1]} {self.real(e[3])})"
        if tag == "un":
            a = self.real(e[2])
            f = e[1]
            if f == "neg":
                return f"(-{a})"
            if f == "abs":
                return f"fabs{'f' if A == 'float' else ''}({a})"
            if f == "sqrt":
                return f"sqrt{'f' if A == 'float' else ''}({a})"
            if f in ("exp", "log", "tanh", "erf", "sin", "cos"):
                return f"ok_{f}{'f' if A == 'float' else ''}({a})"
            raise AssertionError(f)
        if tag == "select":
            return f"({self.boolx(e[1])} ? {self.real(e[2])} : {self.real(e[3])})"
        if tag == "real":
            return f"(({A})(double)({self.intx(e[1])}))"
        if tag == "int":
            return f"(({A})(double)rs_i64((double){self.real(e[1])}))"
        if tag == "cmp":
            return f"(({A})(int64_t)({self.boolx(e)}))"
        raise Refused(f"{tag} in a real position")

    def intx(self, e):
        tag = e[0]
        if tag == "num":
            x = float(e[1])
            if x == int(x) if x == x and abs(x) != float("inf") else False:
                return f"((int64_t){int(x)}LL)"
            return f"rs_i64({_hexlit(x)})"
        if tag == "iv":
            return f"i{e[1]}"
        if tag == "si":
            return f"n{e[1]}"
        if tag == "load":
            b, off = e[1], self.offset(e[1], e[2])
            if self.kinds[b] == "i64":
                return f"p{b}[{off}]"
            return f"rs_i64((double){self.load_stored(b, off)})"
        if tag == "bin" and e[1] in ("+", "*"):
            return f"({self.intx(e[2])} {e[1]} {self.intx(e[3])})"
        if tag == "select":
            return f"({self.boolx(e[1])} ? {self.intx(e[2])} : {self.intx(e[3])})"
        if tag == "int":
            return f"rs_i64((double){self.real(e[1])})"
        # every other expression: its real value, `as i64` (exec.rs:707)
        return f"rs_i64((double){self.real(e)})"

    def boolx(self, e):
        if e[0] == "cmp":
            return f"({self.real(e[2])} {e[1]} {self.real(e[3])})"
        return f"({self.intx(e)} != 0)"

    def vec(self, e):
        """The expression of lane `l`."""
        tag = e[0]
        if tag == "vv":
            return f"v{e[1]}[l]"
        if tag == "vload":
            b, off = e[1], self.offset(e[1], e[2])
            return f"(({self.A}){self.load_stored(b, f'{off} + l')})"
        if tag == "splat":
            return self.real(e[1])
        if tag == "vbin":
            return f"({self.vec(e[2])} {e[1]} {self.vec(e[3])})"
        return self.real(e)

    # ----- statements ----------------------------------------------------------
    def store(self, b, off, val, pad):
        kind, p = self.kinds[b], f"p{b}"
        if kind == "i64":
            return [f"{pad}{p}[{off}] = {val};"]
        if kind in ("f32", "f64"):
            return [f"{pad}{p}[{off}] = {val};"]
        if kind == "bf16":
            return [f"{pad}{p}[{off}] = oc_f32_to_bf16({val});"]
        if kind == "f16":
            return [f"{pad}{{ float t_ = {val}; if (oc_overflows_f16((double)t_)) ovf = 1; {p}[{off}] = oc_f64_to_f16((double)t_); }}"]
        if kind == "e8m15":
            return [f"{pad}{{ float t_ = {val}; if (oc_overflows_e8m15((double)t_)) ovf = 1; st24({p}, {off}, oc_f64_to_e8m15((double)t_)); }}"]
        raise AssertionError(kind)

    def stmts(self, body, depth, out, split_var=None):
        pad = "    " * depth
        for s in body:
            tag = s[0]
            if tag == "for":
                v, n = s[1], s[2]
                if split_var is not None and v == split_var:
                    out.append(f"{pad}for (i{v} = lo; i{v} < hi; i{v}++) {{")
                else:
                    out.append(f"{pad}for (i{v} = 0; i{v} < {n}; i{v}++) {{")
                self.stmts(s[3], depth + 1, out)
                out.append(pad + "}")
            elif tag == "if":
                out.append(f"{pad}if ({self.boolx(s[1])}) {{")
                self.stmts(s[2], depth + 1, out)
                out.append(pad + "}")
            elif tag == "set":
                out.append(f"{pad}s{s[1]} = {self.real(s[2])};")
            elif tag == "seti":
                out.append(f"{pad}n{s[1]} = {self.intx(s[2])};")
            elif tag == "setl":
                out.append(f"{pad}{{ int64_t t_ = {self.intx(s[2])}; i{s[1]} = t_ < 0 ? 0 : t_; }}")
            elif tag == "vset":
                out.append(f"{pad}{{ {self.A} t_[{self.lanes}]; for (int l = 0; l < {self.lanes}; l++) t_[l] = {self.vec(s[2])}; "
                           f"for (int l = 0; l < {self.lanes}; l++) v{s[1]}[l] = t_[l]; }}")
            elif tag == "store":
                b, off = s[1], self.offset(s[1], s[2])
                val = self.intx(s[3]) if self.kinds[b] == "i64" else self.real(s[3])
                out.extend(self.store(b, off, val, pad))
            elif tag == "vstore":
                b, off = s[1], self.offset(s[1], s[2])
                out.append(f"{pad}{{ {self.A} w_[{self.lanes}]; for (int l = 0; l < {self.lanes}; l++) w_[l] = {self.vec(s[3])};")
                out.append(f"{pad}  for (int l = 0; l < {self.lanes}; l++) {{")
                out.extend(self.store(b, f"{off} + l", "w_[l]", pad + "    "))
                out.append(f"{pad}  }} }}")
            else:
                raise AssertionError(tag)

    def program(self, fname):
        k = self.k
        split = parallel_outer(k)
        lines = [f"void {fname}(void *const *bufs, int64_t lo, int64_t hi) {{"]
        ctype = {"f32": "float", "f64": "double", "bf16": "uint16_t", "f16": "uint16_t", "e8m15": "uint8_t", "i64": "int64_t",
                 "q8": "int8_t", "q4": "uint8_t"}
        for i, kind in enumerate(self.kinds):
            lines.append(f"    {ctype[kind]} *restrict p{i} = ({ctype[kind]} *)bufs[{i}];")
        # the scales of the integer inputs after the output, then the flag
        # (crates/presk-cranelift/src/lib.rs:1609-1629)
        for b, (slot, _, _) in self.quant.items():
            lines.append(f"    const float *restrict sc{b} = (const float *)bufs[{slot}];")
        if self.guarded:
            lines.append(f"    uint32_t *flag = (uint32_t *)bufs[{self.n_in + 1 + len(self.quant)}];")
        lines.append("    int ovf = 0; (void)ovf; (void)lo; (void)hi;")
        for v in range(k.nloops):
            lines.append(f"    int64_t i{v} = 0; (void)i{v};")
        for v in range(k.nreal):
            lines.append(f"    {self.A} s{v} = 0; (void)s{v};")
        for v in range(k.nint):
            lines.append(f"    int64_t n{v} = 0; (void)n{v};")
        for v in range(k.nvec):
            lines.append(f"    {self.A} v{v}[{max(self.lanes, 1)}] = {{0}}; (void)v{v};")
        self.stmts(k.body, 1, lines, split_var=k.body[0][1] if split is not None else None)
        if self.guarded:
            lines.append("    if (ovf) __atomic_fetch_or(flag, 1u, __ATOMIC_RELAXED);")
        lines.append("}")
        return "\n".join(lines)


def parallel_outer(k: kt.Kernel):
    """`Kernel::parallel_outer` (ir.rs:336-373): the outermost loop's bound when
    the body is one loop and every store indexes the output with its variable
    directly."""
    if len(k.body) != 1 or k.body[0][0] != "for":
        return None
    var = k.body[0][1]
    state = {"stores": 0, "ok": True}

    def walk(body):
        for s in body:
            tag = s[0]
            if tag == "for":
                walk(s[3])
            elif tag == "if":
                walk(s[2])
            elif tag in ("store", "vstore"):
                state["stores"] += 1
                if not any(e == ("iv", var) for e in s[2]):
                    state["ok"] = False
            elif tag == "setl" and s[1] == var:
                state["ok"] = False

    walk(k.body[0][3])
    return k.body[0][2] if state["ok"] and state["stores"] > 0 else None


PRELUDE = r"""
#include <stdint.h>
#include <math.h>
#include "codes.h"
float ok_expf(float); float ok_logf(float); float ok_tanhf(float); float ok_erff(float);
float ok_sinf(float); float ok_cosf(float);
double ok_exp(double); double ok_log(double); double ok_tanh(double); double ok_erf(double);
double ok_sin(double); double ok_cos(double);
/* Rust's `f as i64`: saturating, NaN to 0 */
static inline int64_t rs_i64(double x) {
    if (x != x) return 0;
    if (x >= 9223372036854775807.0) return INT64_MAX;
    if (x <= -9223372036854775808.0) return INT64_MIN;
    return (int64_t)x;
}
/* int4 weights, two a byte: element e the low nibble of byte e/2 when e is
   even, else the high one, sign-extended (crates/presk-rt/src/quant.rs:333-337) */
static inline int oc_nibble(const uint8_t *p, int64_t e) {
    const int n = (e & 1) ? p[e >> 1] >> 4 : p[e >> 1] & 15;
    return n >= 8 ? n - 16 : n;
}
static inline uint32_t ld24(const uint8_t *p, int64_t e) {
    return (uint32_t)p[3*e] | ((uint32_t)p[3*e+1] << 8) | ((uint32_t)p[3*e+2] << 16);
}
static inline void st24(uint8_t *p, int64_t e, uint32_t c) {
    p[3*e] = (uint8_t)c; p[3*e+1] = (uint8_t)(c >> 8); p[3*e+2] = (uint8_t)(c >> 16);
}
"""

DRIVER = r"""
#include <omp.h>
void run_split(void *const *bufs, int64_t bound, int threads) {
    if (threads <= 1 || bound <= 1) { KFN(bufs, 0, bound); return; }
    if (threads > bound) threads = (int)bound;
    #pragma omp parallel for num_threads(threads) schedule(static, 1)
    for (int w = 0; w < threads; w++) {
        int64_t lo = bound * w / threads, hi = bound * (w + 1) / threads;
        KFN(bufs, lo, hi);
    }
}
"""

_CACHE = os.environ.get("PRESK_ORACLE_CACHE", os.path.join(tempfile.gettempdir(), "presk-oracle-cache"))
_LOADED: dict = {}


def compile_kernel(text: str, dtype: str, lanes: int = 1, opt: str = "-O2", native: bool = False):
    """The C of a kernel, built into a shared object: (library, parsed kernel,
    split bound or None, guarded)."""
    k = kt.parse_kernel(text)
    p = _Printer(k, dtype, lanes)
    src = PRELUDE + p.program("kern") + "\n#define KFN kern\n" + DRIVER
    flags = [opt, "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-fopenmp", "-I", HERE]
    if native:
        flags.append("-march=native")
    key = hashlib.sha1((src + " ".join(flags)).encode()).hexdigest()[:20]
    if key in _LOADED:
        return _LOADED[key], k, parallel_outer(k), p.guarded
    os.makedirs(_CACHE, exist_ok=True)
    so = os.path.join(_CACHE, f"k_{key}.so")
    if not os.path.exists(so):
        # unique temporaries: threads of one process may build the same key
        fd, c = tempfile.mkstemp(suffix=".c", prefix=f"k_{key}_", dir=_CACHE)
        with os.fdopen(fd, "w") as f:
            f.write(src)
        tmp = c[:-2] + ".so.tmp"
        try:
            subprocess.run(["gcc", *flags, "-o", tmp, c, os.path.join(HERE, "libm.c"), "-lm"], check=True, capture_output=True)
            os.replace(tmp, so)
        finally:
            for f in (c, tmp):
                if os.path.exists(f):
                    os.remove(f)
    lib = ctypes.CDLL(so)
    lib.kern.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64, ctypes.c_int64]
    lib.run_split.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64, ctypes.c_int]
    _LOADED[key] = lib
    return lib, k, parallel_outer(k), p.guarded


def quant_of(ty: str):
    """(bits, over, span) of an integer-weight buffer type `int8/1` or
    `int4/1..3` (crates/presk-kernel/src/ir.rs:506-507), else None."""
    m = re.fullmatch(r"int([48])/(\d+)(?:\.\.(\d+))?", ty)
    if not m:
        return None
    over = int(m.group(2))
    return int(m.group(1)), over, (int(m.group(3)) - over) if m.group(3) else 1


def storage_array(ty: str, numel: int) -> np.ndarray:
    """A zeroed buffer of `numel` elements of storage type `ty` (e8m15: 3 bytes each)."""
    if ty == "e8m15":
        return np.zeros(numel * 3, dtype=np.uint8)
    return np.zeros(numel, dtype=NP_STORAGE[ty])


def run(text: str, dtype: str, inputs: list, lanes: int = 1, threads: int = 1, out: np.ndarray | None = None, native: bool = False):
    """Run a kernel on the CPU with the interpreter's semantics.

    `inputs` are numpy arrays holding each input's storage (f32 as float32,
    bf16/f16 as uint16 codes, e8m15 as 3 bytes per element, i64 as int64).
    Returns (output storage array, overflow flag)."""
    lib, k, split, guarded = compile_kernel(text, dtype, lanes, native=native)
    if len(inputs) != len(k.inputs):
        raise ValueError(f"{k.name}: {len(inputs)} inputs for {len(k.inputs)}")
    scales = []
    inputs = list(inputs)
    for i, (a, b) in enumerate(zip(inputs, k.inputs)):
        q = quant_of(b.ty)
        if q is not None:
            # an integer input is (codes, f32 scales)
            a, sc = a
            inputs[i] = a
            scales.append(np.ascontiguousarray(sc, dtype=np.float32))
            want = b.numel if q[0] == 8 else (b.numel + 1) // 2
        else:
            ty = b.ty if b.ty != dtype else dtype
            want = b.numel * (3 if ty == "e8m15" else 1)
        if a.size != want or not a.flags.c_contiguous:
            raise ValueError(f"{k.name}: input %{i} has {a.size} storage elements, {want} expected")
    if out is None:
        out = storage_array(k.output.ty, k.output.numel)
    flag = np.zeros(1, dtype=np.uint32)
    ptrs = [a.ctypes.data for a in inputs] + [out.ctypes.data] + [sc.ctypes.data for sc in scales]
    if guarded:
        ptrs.append(flag.ctypes.data)
    arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
    if split is not None:
        lib.run_split(arr, split, threads)
    else:
        lib.kern(arr, 0, 1)
    return out, bool(flag[0])
