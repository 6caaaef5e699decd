"""Throughput of the executor on one MI355X, with the roofline of its dominant
kernel and the reference's CPU path timed beside it.

    python bench.py [--workload mlp|linear] [--steps K] [--warmup W] [--gpus 1]

A step is one call of the workload's entry over one batch of synthetic,
seeded inputs already resident in HBM: every launch of the program
(presk_amd/configs.py), enqueued on one stream.  Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "tokens/sec course-GPT fwd+bwd; matmul TFLOP/s as % of MFMA peak"
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}   # MI355X dense MFMA
HBM_GBS = 8000.0


def cpu_baseline(workload: str, dtype: str, rows: int, threads: int):
    """The oracle (the kernel interpreter's semantics in C, -O3 -march=native,
    the outermost parallel loop split over OpenMP threads as the native
    executor splits it) on a bounded sample of the workload's rows."""
    import numpy as np

    from oracle import cexec
    from presk_amd import configs

    if workload == "mlp":
        p, host, out, _ = configs.mlp(rows=rows, dtype=dtype)
    else:
        p, host, out, _ = configs.linear(batch=rows, dtype=dtype)
    vals = {}
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, configs._input_specs(ln.low)):
            if name in host and name not in vals:
                vals[name] = configs.encode(host[name].reshape(-1)[:count], ty)
    # compile outside the timed region
    for ln in p.launches:
        cexec.compile_kernel(ln.low.text, ln.low.dtype, ln.low.lanes, opt="-O3", native=True)
    best = None
    for _ in range(2):
        t0 = time.perf_counter()
        env = dict(vals)
        for ln in p.launches:
            env[ln.out], _ = cexec.run(ln.low.text, ln.low.dtype, [env[n] for n in ln.ins], lanes=ln.low.lanes,
                                       threads=threads, native=True)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    return rows / best, best


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="mlp", choices=["mlp", "linear"])
    ap.add_argument("--dtype", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "multi-GPU sharding is a design (DESIGN.md), not a run.", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    from presk_amd import configs, hip

    dtype = args.dtype or ("bf16" if args.workload == "mlp" else "f32")
    if args.workload == "mlp":
        p, host, out, flops = configs.mlp(dtype=dtype)
        tokens, cfg = 8192, {"workload": "config 2: MLP block LN -> Linear 768->3072 -> GELU -> Linear 3072->768 -> residual",
                             "rows": 8192, "d_model": 768, "hidden": 3072, "storage": dtype, "compute": "f32"}
    else:
        p, host, out, flops = configs.linear(dtype=dtype)
        tokens, cfg = 4096, {"workload": "config 1: Linear x.w+b", "batch": 4096, "in": 1024, "out": 1024,
                             "storage": dtype, "compute": "f32"}
    p.compile()
    configs.load_inputs(p, host)
    p.prepare()
    for _ in range(args.warmup):
        p.run()
    hip.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        p.run()
    hip.sync()
    dt = time.perf_counter() - t0
    p.check_overflow()
    ms_step = dt * 1000.0 / args.steps

    # the dominant kernel: the launch with the largest time, timed alone with
    # HIP events on its stream
    times = p.kernel_times(reps=max(args.steps, 10))
    ln, ms = max(times, key=lambda t: t[1])
    c = ln.compiled
    if c.flops > 0:
        achieved = c.flops / (ms * 1e-3) / 1e12
        peak = PEAK_TFLOPS[dtype]
        roof = {"kernel": f"{ln.low.name} [{c.kind}, {c.order}]", "bound": "mfma", "achieved": round(achieved, 2),
                "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None,
                "ms_per_launch": round(ms, 5), "algorithmic_flops": c.flops}
    else:
        achieved = c.bytes / (ms * 1e-3) / 1e9
        roof = {"kernel": f"{ln.low.name} [{c.kind}, {c.order}]", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_GBS, "unit": "GB/s", "frac": round(achieved / HBM_GBS, 4), "traffic": None,
                "ms_per_launch": round(ms, 5), "algorithmic_bytes": c.bytes}
    per_kernel = [{"kernel": l.low.name, "kind": l.compiled.kind, "ms": round(m, 5)} for l, m in times]

    rec = {"metric": METRIC, "value": round(tokens / (ms_step * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,1) inputs, xavier weights)",
           "config": cfg, "matmul_tflops": round(flops / (ms_step * 1e-3) / 1e12, 2), "roofline": roof,
           "kernels": per_kernel}
    if not args.no_cpu:
        threads = min(os.cpu_count() or 1, 16)
        rows = args.cpu_rows or (4096 if args.workload == "mlp" else 1024)
        v, secs = cpu_baseline(args.workload, dtype, rows, threads)
        rec["cpu_baseline"] = {"value": round(v, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
                               "sample": f"{rows} of {tokens} rows of the same workload, oracle C restatement "
                                         f"(-O3 -march=native, OpenMP outer-loop split), best of 2: {secs:.2f} s"}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
