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
DATA = {"gpt-step": "synthetic (seeded ids and targets uniform over the vocabulary, N(0,0.02) weights)",
        "gpt-forward": "synthetic (seeded ids and targets uniform over the vocabulary, N(0,0.02) weights)",
        "llama": "synthetic (ids uniform over the vocabulary; N(0,0.02) weights drawn on the device, "
                 "presk_hip_fill_normal)"}


def workload(name: str, dtype: str, rows=None, realize=None, dropout=0.0, adamw=False):
    """(program, host inputs, tokens per step, contraction flops, config record)
    of a workload; `rows` shrinks it for the CPU sample; `realize` (`@FILE`)
    gives the GPT's sites their storage types (a mixed realization).  The
    Llama forward's inputs are made on the device (`host` None).  `adamw`:
    the training step followed by its optimizer step (adamw.step at step
    200 of 1000, 05_gpt.psk's hyperparameters)."""
    from presk_amd import configs, gpt, llama
    from presk_amd.realize import Realization

    if name == "llama":
        s = llama.LLAMA_7B
        p, _, _ = llama.build(s, dtype)
        cfg = {"workload": "config 5: Llama-7B-shaped decoder forward (logits of a full context, as presk serve "
                           "recomputes them)", "L": s.L, "d_model": s.D, "heads": s.H, "kv_heads": s.G, "ffn": s.FF,
               "vocab": s.V, "batch": s.B, "seq": s.T, "rope_base": s.base, "rmsnorm_eps": s.eps, "storage": dtype,
               "compute": "f32", "params": llama.param_count(s), "launches": len(p.launches)}
        return p, None, s.B * s.T, llama.contraction_flops(s), cfg

    if name == "mlp":
        r = rows or 8192
        p, host, _, flops = configs.mlp(rows=r, dtype=dtype)
        cfg = {"workload": "config 2: MLP block LN -> Linear 768->3072 -> GELU -> Linear 3072->768 -> residual",
               "rows": r, "d_model": 768, "hidden": 3072, "storage": dtype, "compute": "f32"}
        return p, host, r, flops, cfg
    if name == "linear":
        r = rows or 4096
        p, host, _, flops = configs.linear(batch=r, dtype=dtype)
        cfg = {"workload": "config 1: Linear x.w+b", "batch": r, "in": 1024, "out": 1024, "storage": dtype, "compute": "f32"}
        return p, host, r, flops, cfg
    train = name == "gpt-step"
    s = gpt.COURSE if rows is None else gpt.GptShape(B=max(rows // gpt.COURSE.T, 1))
    r = Realization.parse(realize) if realize else None
    opt = bool(adamw and train)
    p, b, names = gpt.build(s, dtype, train=train, realize=r, dropout=dropout if train else 0.0, optimizer=opt)
    host = gpt.host_inputs(s)
    if opt:
        host.update(gpt.optimizer_inputs(s, 200, 1000))
    cfg = {"workload": ("config 4: course GPT training step (loss value and gradient of every parameter)" if train
                        else "config 3: course GPT forward and loss"),
           "L": s.L, "d_model": s.D, "heads": s.H, "vocab": s.V, "batch": s.B, "seq": s.T,
           "storage": dtype if r is None else f"mixed ({realize})", "compute": "f32", "launches": len(p.launches),
           "dropout": dropout if train else 0.0, "optimizer": "adamw" if opt else None}
    return p, host, s.B * s.T, gpt.contraction_flops(s, train), cfg


def launch_key(ln) -> str:
    """A launch as the traffic table names it: its kernel's header (name and
    shapes) and the class and order it runs in."""
    c = ln.compiled
    return f"{ln.low.text.splitlines()[0].rstrip(' {')} | {c.kind} {c.order}"


def _traffic_table() -> dict:
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, then
    WRITE_SIZE, each scaled by the copy probe's reading), as committed in
    profiles/traffic.json: {launch key: bytes}."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return {e["key"]: e["bytes_per_launch"] for e in json.load(f)["launches"]}
    except (OSError, ValueError, KeyError):
        return {}


TRAFFIC = _traffic_table()


def copy_probe():
    """neg over 64 Mi f32 (256 MiB read, 256 MiB written), three launches."""
    from presk_amd import hip, lower as L
    hip.init(0)
    x = L.Operand(L.ax(("rows", 16384), ("cols", 4096)))
    low = L.unary("neg", [x], "f32")
    c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    n = 16384 * 4096
    a, b = hip.DeviceBuffer(4 * n), hip.DeviceBuffer(4 * n)
    a.zero()
    for _ in range(3):
        c.run([a.ptr, b.ptr])
    hip.sync()
    print(json.dumps({"copy_probe": low.name, "bytes_read": 4 * n, "bytes_written": 4 * n, "runs": 3}), flush=True)


def cpu_baseline(name: str, dtype: str, rows: int, threads: int, realize=None, dropout=0.0, adamw=False):
    """The oracle (the kernel interpreter's semantics in C, -O3 -march=native,
    the outermost parallel loop split over OpenMP threads as the native
    executor splits it) on a bounded sample of the workload's rows."""
    from tests import cpu_program

    p, host, tokens, _, _ = workload(name, dtype, rows, realize, dropout, adamw)
    cpu_program.compile_all(p, native=True, workers=threads)
    best = None
    for _ in range(1 if name.startswith("gpt") else 2):
        t0 = time.perf_counter()
        cpu_program.run(p, host, threads=threads, native=True)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    return tokens / best, best, tokens


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="gpt-step", choices=["gpt-step", "gpt-forward", "mlp", "linear", "llama"])
    ap.add_argument("--dtype", default=None)
    ap.add_argument("--realize", default=None, metavar="@FILE",
                    help="a realization file (the reference's schema) for the GPT workloads: storage type per site")
    ap.add_argument("--adamw", action="store_true",
                    help="config 4 with its optimizer step (adamw.step): the training run's whole step")
    ap.add_argument("--dropout", type=float, default=0.0,
                    help="the training step's dropout rate (the course's 0.2): masks drawn on the device, a new "
                         "step key each step")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="issue the launches one by one instead of one HIP graph")
    ap.add_argument("--dominant-only", type=int, default=0, metavar="N",
                    help="after the timing pass, run the dominant launch alone N times and exit (for rocprofv3 --pmc)")
    ap.add_argument("--dominant-match", default=None, metavar="TEXT",
                    help="take the dominant launch among those whose key contains TEXT (counter runs distort "
                         "the timings the choice is made on)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run a plain copy-like nest (neg over 64 Mi f32) 3 times and exit: the counters' calibration")
    ap.add_argument("--cpu-rows", type=int, default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "multi-GPU sharding is a design (DESIGN.md), not a run.", file=sys.stderr)
        sys.exit(2)

    from presk_amd import configs, hip

    if args.copy_probe:
        copy_probe()
        return
    dtype = args.dtype or ("bf16" if args.workload in ("mlp", "llama") else "f32")
    p, host, tokens, flops, cfg = workload(args.workload, dtype, realize=args.realize, dropout=args.dropout, adamw=args.adamw)
    # a training run's keys: step i draws from Key::child(run key, i); the site
    # keys are derived before the timed region, uploaded (608 bytes) each step
    step_keys = []
    if p.masks:
        from presk_amd import gpt, keys
        run_key = keys.from_seed(0)
        step_keys = [gpt.site_keys(gpt.COURSE, keys.child(run_key, i)) for i in range(args.warmup + args.steps)]
    p.compile()
    if host is None:
        from presk_amd import llama
        llama.load_device_inputs(p, llama.LLAMA_7B)
    else:
        configs.load_inputs(p, host)
    p.prepare()
    if not args.eager:
        # the step's 587 launches recorded once and replayed as one HIP graph
        p.record(graph=True)
    for i in range(args.warmup):
        if step_keys:
            p.set_keys(step_keys[i])
        p.run()
    hip.sync()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if step_keys:
            p.set_keys(step_keys[args.warmup + i])
        p.run()
    hip.sync()
    dt = time.perf_counter() - t0
    p.check_overflow()
    ms_step = dt * 1000.0 / args.steps

    # the dominant kernel: the launch with the largest time, timed alone with
    # HIP events on its stream
    times = p.kernel_times(reps=max(args.steps, 10))
    pool = [t for t in times if args.dominant_match is None or args.dominant_match in launch_key(t[0])] or times
    ln, ms = max(pool, key=lambda t: t[1])
    c = ln.compiled
    key = launch_key(ln)
    if args.dominant_only:
        hip.sync()
        for _ in range(args.dominant_only):
            hip.check(hip.lib().presk_hip_run(c.handle, ln.table, 0, max(c.split_bound, 0), None))
        hip.sync()
        print(json.dumps({"dominant": key, "runs": args.dominant_only}), flush=True)
        return
    traffic = TRAFFIC.get(key)
    if c.flops > 0:
        achieved = c.flops / (ms * 1e-3) / 1e12
        peak = PEAK_TFLOPS[ln.low.dtype]
        roof = {"kernel": f"{ln.low.name} [{c.kind}, {c.order}]", "bound": "mfma", "achieved": round(achieved, 2),
                "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                "ms_per_launch": round(ms, 5), "algorithmic_flops": c.flops}
    else:
        achieved = c.bytes / (ms * 1e-3) / 1e9
        roof = {"kernel": f"{ln.low.name} [{c.kind}, {c.order}]", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_GBS, "unit": "GB/s", "frac": round(achieved / HBM_GBS, 4), "traffic": traffic,
                "ms_per_launch": round(ms, 5), "algorithmic_bytes": c.bytes}
    # per nest name: launches and total ms (the step's time by kind of nest)
    agg = {}
    for l, m in times:
        e = agg.setdefault(l.low.name, {"kernel": l.low.name, "kind": l.compiled.kind, "launches": 0, "ms": 0.0})
        e["launches"] += 1
        e["ms"] += m
    per_kernel = sorted(agg.values(), key=lambda e: -e["ms"])[:16]
    for e in per_kernel:
        e["ms"] = round(e["ms"], 4)

    cfg = dict(cfg, launch="eager" if args.eager else "hip graph")
    # the contractions' time at the MFMA peak of each one's storage type over
    # the step's time: flops / peak for one type, weighted for a mixed one
    bound_ms = sum(l.compiled.flops / (PEAK_TFLOPS.get(l.low.dtype, PEAK_TFLOPS["f32"]) * 1e12) * 1e3
                   for l in p.launches if l.compiled.kind == "gemm")
    metric = {"gpt-step": METRIC, "gpt-forward": "tokens/sec course-GPT forward and loss (config 3)",
              "llama": "tokens/sec Llama-7B-shaped forward (config 5); matmul TFLOP/s as % of MFMA peak"}.get(
        args.workload, f"rows/sec {args.workload} (a supplementary workload)")
    rec = {"metric": metric, "value": round(tokens / (ms_step * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": DATA.get(args.workload, "synthetic (seeded N(0,1) inputs, xavier weights)"),
           "config": cfg, "matmul_tflops": round(flops / (ms_step * 1e-3) / 1e12, 2),
           "matmul_frac_of_peak": round(bound_ms / ms_step, 4), "roofline": roof,
           "kernels": per_kernel}
    if not args.no_cpu:
        threads = min(os.cpu_count() or 1, 16)
        rows = args.cpu_rows or {"mlp": 4096, "linear": 1024, "gpt-step": 2048, "gpt-forward": 4096}[args.workload]
        v, secs, n = cpu_baseline(args.workload, dtype, rows, threads, args.realize, args.dropout, args.adamw)
        rec["cpu_baseline"] = {"value": round(v, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
                               "sample": f"{n} of {tokens} tokens (rows) of the same workload: the oracle's C restatement of "
                                         f"the same default-layout nests (-O3 -march=native, -ffp-contract=off, sequential "
                                         f"sums, the outermost parallel loop split over OpenMP threads): {secs:.2f} s"}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
