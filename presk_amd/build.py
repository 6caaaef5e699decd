"""Builds presk_amd/libpresk_hip.so: the executor's C ABI (include/presk_hip.h)
with its hand-written gfx950 kernels, compiled with hipcc for gfx950 only.

    python -m presk_amd.build          # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "libpresk_hip.so")
BUILD = os.path.join(PKG, "_build")

SOURCES = ["ir.cpp", "hipgen.cpp", "presk_hip.cpp", "selftest.hip", "classes.hip", "gemm.hip", "reduce.hip", "rows.hip", "wrows.hip", "scatter.hip", "convert.hip", "synth.hip", "probe.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# f32 semantics the parity rests on: no contraction into FMA, IEEE denormals,
# correctly rounded division and square root; packed-f32 instructions off.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
         "-fno-gpu-flush-denormals-to-zero", "-fhip-fp32-correctly-rounded-divide-sqrt",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", CSRC, "-I", os.path.join(ROOT, "include"), "-Wall", "-Wno-unused-function"]


def _devfmt_inc():
    """devfmt.hpp as a C++ string literal, for the hiprtc builds."""
    text = open(os.path.join(CSRC, "devfmt.hpp")).read()
    body = 'R"PRESKDEVFMT(' + text + ')PRESKDEVFMT"\n'
    path = os.path.join(CSRC, "_devfmt.inc")
    if not os.path.exists(path) or open(path).read() != body:
        with open(path, "w") as f:
            f.write(body)


def _compile(src: str) -> str:
    os.makedirs(BUILD, exist_ok=True)
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> str:
    """Compiles every source and links the library; returns its path."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found: the executor is built for gfx950 with hipcc")
    _devfmt_inc()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + f".tmp{os.getpid()}"
    r = subprocess.run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs,
                        "-L/opt/rocm/lib", "-lhiprtc", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, OUT)
    if verbose:
        h = hashlib.sha1(open(OUT, "rb").read()).hexdigest()[:12]
        print(f"built {OUT} ({os.path.getsize(OUT)} bytes, sha1 {h})")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
