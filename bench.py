"""Throughput of the executor on one MI355X, with the roofline of its dominant
kernel and the reference's CPU path timed beside it.

    python bench.py [--workload mlp|linear] [--steps K] [--warmup W] [--gpus 1]

A step is one call of the workload's entry over one batch of synthetic,
seeded inputs already resident in HBM: every launch of the program
(presk_amd/configs.py), enqueued on one stream.  Prints one JSON line.
"""
from __future__ import annotations

import argparse
import gc
import hashlib
import json
import os
import statistics
import subprocess
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


def source_sha() -> str:
    """sha1 of the executor's device sources: a traffic figure measured on
    other sources is stale."""
    h = hashlib.sha1()
    csrc = os.path.join(ROOT, "presk_amd", "csrc")
    for f in sorted(os.listdir(csrc)):
        if f.endswith((".hip", ".cpp", ".hpp")):
            with open(os.path.join(csrc, f), "rb") as fh:
                h.update(f.encode() + fh.read())
    return h.hexdigest()[:16]


def _traffic_table() -> dict:
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, then
    WRITE_SIZE, each scaled by the copy probe's reading), as committed in
    profiles/traffic.json: {launch key: bytes}, empty when the table was
    measured on other device sources than these."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        if t.get("src_sha") != source_sha():
            return {}
        return {e["key"]: e["bytes_per_launch"] for e in t["launches"]}
    except (OSError, ValueError, KeyError):
        return {}


def measured_peaks() -> dict:
    """The peaks measured on this device, reported beside the vendor's
    nominal ones: the matrix cores' rate in independent MFMA loops (eight
    waves on every CU, nothing else issued; presk_hip_mfma_probe) and the
    HBM rate of a plain copy nest (neg over 64 Mi f32: 256 MiB read and 256
    MiB written a launch, more than the Infinity Cache holds; HIP events over
    10 launches after 2)."""
    import ctypes
    from presk_amd import hip, lower as L
    hip.init(0)
    lib = hip.lib()
    out = {}
    for ty in ("bf16", "f32"):
        ms, fl = ctypes.c_double(), ctypes.c_double()
        hip.check(lib.presk_hip_mfma_probe(ty.encode(), 20000, None, ctypes.byref(ms), ctypes.byref(fl)))
        out[f"mfma_{ty}_tflops"] = round(fl.value / (ms.value * 1e-3) / 1e12, 1)
    x = L.Operand(L.ax(("rows", 16384), ("cols", 4096)))
    low = L.unary("neg", [x], "f32")
    c = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    n = 16384 * 4096
    a, b = hip.DeviceBuffer(4 * n), hip.DeviceBuffer(4 * n)
    a.zero()
    tab = (ctypes.c_void_p * 2)(a.ptr, b.ptr)
    ms = ctypes.c_double()
    hip.check(lib.presk_hip_time(c.handle, tab, 0, max(c.split_bound, 0), None, 2, 10, ctypes.byref(ms)))
    out["hbm_copy_gbs"] = round(8 * n / (ms.value * 1e-3) / 1e9, 1)
    out["probe"] = ("MFMA: v_mfma_f32_32x32x16_bf16 / v_mfma_f32_16x16x4_f32 loops, 8 waves a CU, 8 accumulators "
                    "a wave; HBM: neg over f32[16384, 4096], bytes read + written over time")
    return out


def with_measured(roof: dict, storage: str, peaks) -> dict:
    """The roofline beside the measured peak of its bound (the vendor figure
    stays `peak` and `frac`)."""
    if not peaks:
        return roof
    if roof["bound"] == "mfma":
        pm = peaks["mfma_bf16_tflops" if storage in ("bf16", "f16") else "mfma_f32_tflops"]
    else:
        pm = peaks["hbm_copy_gbs"]
    return dict(roof, peak_measured=pm, frac_of_measured=round(roof["achieved"] / pm, 4))


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


def cpu_child(name, dtype, rows, threads, core, realize, dropout, adamw):
    """One timed call of the oracle's C restatement in this process (a child
    of bench.py, started before the GPU is touched), its kernels loaded from
    the oracle's build cache first; prints {"secs": .., "tokens": ..}."""
    if core >= 0:
        os.sched_setaffinity(0, {core})
    from tests import cpu_program
    p, host, tokens, _, _ = workload(name, dtype, rows, realize, dropout, adamw)
    cpu_program.compile_all(p, native=True, workers=threads)
    t0 = time.perf_counter()
    cpu_program.run(p, host, threads=threads, native=True)
    secs = time.perf_counter() - t0
    print(json.dumps({"secs": secs, "tokens": tokens}), flush=True)


def cpu_baseline(name, dtype, rows_all, rows_one, realize=None, dropout=0.0, adamw=False, repeats=3):
    """The oracle (the kernel interpreter's semantics in C, -O3
    -march=native, sequential sums, the outermost parallel loop split over
    OpenMP threads as the native executor splits it) on bounded samples of
    the workload: `repeats` processes on every host core (capped at 16), one
    after another, and `repeats` one-core processes side by side, each on a
    core of its own.  The median and the best of each, as the reference's
    `presk bench` reports (crates/presk-driver/src/bench.rs:28-48), over
    separate processes (docs/kernels-roadmap.md:482-484).  Runs before the
    GPU is touched."""
    from tests import cpu_program
    cores = sorted(os.sched_getaffinity(0))
    threads = min(len(cores), 16)
    # the kernels compiled once, into the oracle's disk cache the children read
    for rows in (rows_all, rows_one):
        p, _, _, _, _ = workload(name, dtype, rows, realize, dropout, adamw)
        cpu_program.compile_all(p, native=True, workers=threads)

    def child(rows, th, core):
        cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child", str(rows), str(th), str(core),
               "--workload", name, "--dtype", dtype, "--dropout", str(dropout)]
        if realize:
            cmd += ["--realize", realize]
        if adamw:
            cmd.append("--adamw")
        env = dict(os.environ, OMP_NUM_THREADS=str(th))
        return subprocess.Popen(cmd, stdout=subprocess.PIPE, text=True, env=env)

    def collect(procs):
        out = []
        for pr in procs:
            text, _ = pr.communicate()
            if pr.returncode != 0:
                raise RuntimeError(f"cpu baseline child failed ({pr.returncode})")
            out.append(json.loads(text.strip().splitlines()[-1]))
        return out

    # one untimed process first: the first of a run has measured twice as
    # long as those after it (the host's first touch of its memory and
    # caches), which a three-process median would otherwise carry
    warm = collect([child(rows_all, threads, -1)])[0]
    every = [collect([child(rows_all, threads, -1)])[0] for _ in range(repeats)]
    one = collect([child(rows_one, 1, cores[(i * 2) % len(cores)]) for i in range(repeats)])

    def summary(rs):
        rates = sorted(r["tokens"] / r["secs"] for r in rs)
        return statistics.median(rates), rates[-1], rs[0]["tokens"], [round(r["secs"], 3) for r in rs]

    med, best, toks, secs = summary(every)
    med1, best1, toks1, secs1 = summary(one)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(med, 1), "best": round(best, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": model, "repeats": repeats,
            "sample": f"{toks} tokens of the same workload (B {max(toks // 256, 1)} x T 256), {repeats} processes "
                      f"({secs} s a call) after an untimed one ({round(warm['secs'], 3)} s): the oracle's C restatement of the same nests (-O3 -march=native, "
                      f"-ffp-contract=off, sequential sums, the outermost parallel loop split over {threads} OpenMP "
                      f"threads); value = the median, best = the fastest",
            "one_core": {"value": round(med1, 2), "best": round(best1, 2), "unit": "tokens/s", "cores": 1,
                         "sample": f"{toks1} tokens, {repeats} one-thread processes side by side on separate cores "
                                   f"({secs1} s a call)"}}


def measure(name, dtype, steps, warmup, realize=None, dropout=0.0, adamw=False, eager=False, dominant_match=None,
            peaks=None):
    """Times one workload: its launches as one HIP graph (or eager), W untimed
    calls, K timed between synchronizations; then each launch alone with HIP
    events on its stream, the slowest giving the roofline.  Returns
    (record, program, the dominant launch)."""
    from presk_amd import configs, hip
    p, host, tokens, flops, cfg = workload(name, dtype, realize=realize, dropout=dropout, adamw=adamw)
    step_keys = []
    if p.masks:
        from presk_amd import gpt, keys
        run_key = keys.from_seed(0)
        step_keys = [gpt.site_keys(gpt.COURSE, keys.child(run_key, i)) for i in range(warmup + steps)]
    p.compile()
    if host is None:
        from presk_amd import llama
        llama.load_device_inputs(p, llama.LLAMA_7B)
    else:
        configs.load_inputs(p, host)
    p.prepare()
    if not eager:
        p.record(graph=True)
    for i in range(warmup):
        if step_keys:
            p.set_keys(step_keys[i])
        p.run()
    hip.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        if step_keys:
            p.set_keys(step_keys[warmup + i])
        p.run()
    hip.sync()
    dt = time.perf_counter() - t0
    p.check_overflow()
    ms_step = dt * 1000.0 / steps
    times = p.kernel_times(reps=max(min(steps, 20), 10))
    pool = [t for t in times if dominant_match is None or dominant_match in launch_key(t[0])] or times
    ln, ms = max(pool, key=lambda t: t[1])
    c = ln.compiled
    traffic = TRAFFIC.get(launch_key(ln))
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
    if traffic is None:
        roof["traffic_note"] = "no counter measurement of this kernel on these device sources (profiles/traffic.json)"
    roof = with_measured(roof, ln.low.dtype, peaks)
    agg = {}
    for l, m in times:
        e = agg.setdefault(l.low.name, {"kernel": l.low.name, "kind": l.compiled.kind, "launches": 0, "ms": 0.0})
        e["launches"] += 1
        e["ms"] += m
    per_kernel = sorted(agg.values(), key=lambda e: -e["ms"])[:16]
    for e in per_kernel:
        e["ms"] = round(e["ms"], 4)
    # the contractions' time at the MFMA peak of each one's storage type
    bound_ms = sum(l.compiled.flops / (PEAK_TFLOPS.get(l.low.dtype, PEAK_TFLOPS["f32"]) * 1e12) * 1e3
                   for l in p.launches if l.compiled.kind == "gemm")
    cfg = dict(cfg, launch="eager" if eager else "hip graph")
    rec = {"value": round(tokens / (ms_step * 1e-3), 1), "unit": "tokens/s", "steps": steps, "warmup": warmup,
           "ms_per_step": round(ms_step, 4), "dtype": dtype if realize is None else "mixed", "config": cfg,
           "matmul_tflops": round(flops / (ms_step * 1e-3) / 1e12, 2), "matmul_frac_of_peak": round(bound_ms / ms_step, 4),
           "roofline": roof, "kernels": per_kernel, "kernel_ms_sum": round(sum(m for _, m in times), 4)}
    return rec, p, (ln, c)


def _rotated_ms(ln, ring_bytes: float, min_ms: float = 3.0) -> tuple:
    """Mean ms of one launch over copies of its buffers that together exceed
    the MI355X's 256 MB Infinity Cache: R copies of every input (their
    contents copied from the launch's own) and of the output, launched in
    turn as one recorded sequence, repeated until at least `min_ms` has run,
    so that a launch whose working set the cache would hold reads HBM as it
    does inside a step.  Returns (ms, R)."""
    import ctypes

    import numpy as np

    from presk_amd import hip
    from presk_amd.configs import _input_specs
    lib = hip.lib()
    c = ln.compiled
    specs = _input_specs(ln.low)
    sizes = [max(cnt, 1) * hip.STORAGE_BYTES[ty] for ty, cnt in specs]
    n_out = 1
    for a in ln.low.out_axes:
        n_out *= a.len
    out_bytes = max(n_out, 1) * hip.STORAGE_BYTES["i64" if ln.low.out_kind == "idx" else ln.low.dtype]
    ws = sum(sizes) + out_bytes
    r = max(1, min(32, int(-(-ring_bytes // max(ws, 1)))))
    ptrs = [ln.table[i] for i in range(len(ln.table))]
    host = []
    for i, nb in enumerate(sizes):
        a = np.empty(nb, np.uint8)
        hip.check(lib.presk_hip_d2h(a.ctypes.data, ptrs[i], nb, None))
        host.append(a)
    keep, tables = [], []
    for _ in range(r):
        bufs = [hip.DeviceBuffer.of(a) for a in host] + [hip.DeviceBuffer(out_bytes)]
        keep.append(bufs)
        t = [b.ptr for b in bufs] + ptrs[len(sizes) + 1:]
        tables.append((ctypes.c_void_p * len(t))(*t))
    b = ctypes.c_void_p()
    hip.check(lib.presk_hip_batch_create(ctypes.byref(b)))
    try:
        for t in tables:
            hip.check(lib.presk_hip_batch_add(b, c.handle, t, 0, max(c.split_bound, 0)))
        hip.check(lib.presk_hip_batch_graph_branches(b, 1))
        for _ in range(2):
            hip.check(lib.presk_hip_batch_run(b, None))
        hip.sync()
        reps, spent = 1, 0.0
        while True:
            t0 = time.perf_counter()
            for _ in range(reps):
                hip.check(lib.presk_hip_batch_run(b, None))
            hip.sync()
            spent = (time.perf_counter() - t0) * 1e3
            if spent >= min_ms:
                break
            reps *= 2
        return spent / (reps * r), r
    finally:
        lib.presk_hip_batch_release(b)
        del keep


def per_launch_table(p, path, ring_mb: float = 768.0):
    """Each distinct launch of the step (by kernel text) timed alone over a
    ring of copies of its buffers larger than the Infinity Cache (_rotated_ms),
    so that "% of HBM" measures HBM: its count, mean time, algorithmic bytes
    (inputs and output once) and flops, and the rates they give against the
    HBM and MFMA peaks; written to `path` as markdown rows, slowest total
    first."""
    from presk_amd import hip
    hip.sync()
    agg = {}
    for ln in p.launches:
        head = ln.low.text.split("{")[0].strip()
        e = agg.setdefault(head, [0, 0.0, ln, 1])
        e[0] += 1
    for i, (head, e) in enumerate(agg.items()):
        ms, r = _rotated_ms(e[2], ring_mb * 1e6)
        e[1], e[3] = ms * e[0], r
        print(f"[per-launch] {i + 1}/{len(agg)} {ms * 1e3:.1f} us over {r} copies: {head[:90]}", file=sys.stderr, flush=True)
    total = sum(e[1] for e in agg.values())
    rows = ["| launch (kernel text's head) | class, order | launches | copies | us each | us a step | MB | GB/s | % of HBM | TFLOP/s | % of MFMA |",
            "|---|---|---|---|---|---|---|---|---|---|---|"]
    for head, (n, ms, ln, r) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        c = ln.compiled
        each = ms / n * 1e-3
        gbs = c.bytes / each / 1e9
        tf = c.flops / each / 1e12 if c.flops else 0.0
        peak = PEAK_TFLOPS.get(ln.low.dtype, PEAK_TFLOPS["f32"])
        rows.append(f"| `{head[:160]}` | {c.kind}, {c.order} | {n} | {r} | {each * 1e6:.2f} | {ms * 1e3:.1f} | {c.bytes / 1e6:.1f} | "
                    f"{gbs:.0f} | {100 * gbs / HBM_GBS:.0f} | " + (f"{tf:.1f} | {100 * tf / peak:.0f} |" if c.flops else "| |"))
    rows.append(f"| (all {sum(e[0] for e in agg.values())} launches) | | | | | {total * 1e3:.1f} | | | | | |")
    with open(path, "w") as f:
        f.write("\n".join(rows) + "\n")


# the workloads whose distinct launches the traffic table covers
TRAFFIC_WORKLOADS = [("gpt-step", "f32", None), ("gpt-step", "bf16", None),
                     ("gpt-forward", "f32", "@" + os.path.join(ROOT, "presk_amd", "realizations", "course_gpt_mixed.json")),
                     ("linear", "f32", None), ("mlp", "bf16", None), ("llama", "bf16", None)]


def traffic_run(keys_path):
    """The counter runs' program (under rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): the copy probe (neg over 64 Mi f32), then every distinct
    launch of TRAFFIC_WORKLOADS 3 times.  Each region of dispatches follows
    one launch of a marker nest (a one-element copy named `traffic_mark`,
    found by name in the counter table): the probe's, each workload's set-up
    and first run (key `__setup__`, left out of the table) and each launch's
    group; the keys, in order, and the device sources' sha go to
    `keys_path` for traffic_table."""
    from presk_amd import configs, hip, llama, lower as L
    lib = hip.lib()
    hip.init(0)
    keys = []
    one = L.unary("neg", [L.Operand(L.ax(("one", 1)))], "f32")
    mark = hip.Compiled(one.text.replace("kernel neg ", "kernel traffic_mark ", 1), "f32", one.lanes, hip.FAST)
    mbuf = [hip.DeviceBuffer(256), hip.DeviceBuffer(256)]

    def marker(key):
        mark.run([mbuf[0].ptr, mbuf[1].ptr])
        keys.append(key)

    x = L.Operand(L.ax(("rows", 16384), ("cols", 4096)))
    low = L.unary("neg", [x], "f32")
    cp = hip.Compiled(low.text, "f32", low.lanes, hip.FAST)
    a, b = hip.DeviceBuffer(4 << 26), hip.DeviceBuffer(4 << 26)   # contents as allocated: neg moves them all
    marker("__copy_probe__")
    for _ in range(3):
        cp.run([a.ptr, b.ptr])
    hip.sync()
    del a, b
    for name, dt, real in TRAFFIC_WORKLOADS:
        marker("__setup__")
        p, host, _, _, _ = workload(name, dt, realize=real)
        p.compile()
        if host is None:
            llama.load_device_inputs(p, llama.LLAMA_7B)
        else:
            configs.load_inputs(p, host)
        p.prepare()
        p.run()
        hip.sync()
        seen = set()
        for ln in p.launches:
            k = launch_key(ln)
            if k in seen:
                continue
            seen.add(k)
            c = ln.compiled
            marker(k)
            for _ in range(3):
                hip.check(lib.presk_hip_run(c.handle, ln.table, 0, max(c.split_bound, 0), None))
        hip.sync()
        print(f"[traffic] {name} {dt}: {len(seen)} distinct launches", file=sys.stderr, flush=True)
        del p
        gc.collect()
    marker("__end__")
    hip.sync()
    with open(keys_path, "w") as f:
        json.dump({"keys": keys, "src_sha": source_sha()}, f)
    print(f"[traffic] {len(keys)} regions", file=sys.stderr, flush=True)


def traffic_table(keys_path, fetch_glob, write_glob, out_path):
    """profiles/traffic.json from the two counter runs of traffic_run: the
    per-dispatch FETCH_SIZE and WRITE_SIZE (KiB) split into regions at the
    marker launches, each launch's 3 calls averaged, every KiB scaled by the
    bytes the copy probe moves per KiB its region counts."""
    import csv
    import glob

    with open(keys_path) as f:
        keys = json.load(f)

    def groups(pattern, counter):
        rows = []
        for path in glob.glob(pattern, recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    if r.get("Counter_Name") == counter:
                        rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        rows.sort()
        # a region: the dispatches after one marker launch, up to the next
        # (the runtime's own copy and fill kernels left out)
        segs = []
        for _, kname, v in rows:
            if kname.startswith("pk_traffic_mark"):
                segs.append([])
            elif segs and not kname.startswith("__amd_rocclr"):
                segs[-1].append(v)
        return segs

    fetch, write = groups(fetch_glob, "FETCH_SIZE"), groups(write_glob, "WRITE_SIZE")
    k = keys["keys"]
    if len(fetch) != len(k) or len(write) != len(k):
        raise SystemExit(f"traffic_table: {len(k)} regions expected, {len(fetch)} / {len(write)} found")
    probe = 4 << 26
    ff = probe / (sum(fetch[0]) / 3 * 1024)
    wf = probe / (sum(write[0]) / 3 * 1024)
    out = []
    for i, key in enumerate(k):
        if key.startswith("__"):
            continue
        fb = sum(fetch[i]) / 3 * 1024 * ff
        wb = sum(write[i]) / 3 * 1024 * wf
        out.append({"key": key, "bytes_per_launch": round(fb + wb), "fetch_bytes": round(fb), "write_bytes": round(wb),
                    "dispatches": len(fetch[i]) // 3})
    with open(out_path, "w") as f:
        json.dump({"src_sha": keys["src_sha"],
                   "method": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over bench.py --traffic-run (every distinct "
                             "launch of the workloads 3 times after a marker launch), each KiB scaled by the copy "
                             f"probe's reading (neg over 64 Mi f32: FETCH x {ff:.3f}, WRITE x {wf:.3f})",
                   "launches": out}, f, indent=1)
    print(f"[traffic] wrote {out_path}: {len(out)} launches; copy probe factors {ff:.3f} {wf:.3f}", file=sys.stderr)


# the contractions of the configurations, [M x K] . [K x N]: Llama's
# projections and head, the MLP block's two, the course step's three
YARDSTICK_SHAPES = [(2048, 4096, 4096), (2048, 11008, 4096), (2048, 4096, 11008), (2048, 32000, 4096),
                    (8192, 3072, 768), (8192, 768, 3072), (16384, 384, 384), (16384, 1536, 384), (16384, 384, 1536)]


def yardstick(path, ring_mb: float = 600.0):
    """The vendor library beside this executor on the same contractions: each
    shape of YARDSTICK_SHAPES in bf16 and f32 (row-major [M x K] . [K x N],
    a `dot`), timed as torch.matmul (hipBLASLt on this image) and as this
    executor's contraction, both over rings of operand copies larger than
    the Infinity Cache: the library's 30 back-to-back calls after 3 untimed
    ones between HIP events, the executor's ring recorded as one graph and
    replayed 8 times under the host clock; written to `path` as a markdown
    table.  A yardstick of
    what the hardware gives a tuned library on these shapes, not a path of
    this executor."""
    import ctypes

    import torch

    from presk_amd import hip, lower as L
    hip.init(0)
    dev = torch.device("cuda:0")
    rows = ["| shape M x N x K | type | hipBLASLt (torch.matmul) us | TFLOP/s | % of peak | this executor us | TFLOP/s | % of peak | order |",
            "|---|---|---|---|---|---|---|---|---|"]
    for dt in ("bf16", "f32"):
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        esz = 2 if dt == "bf16" else 4
        peak = PEAK_TFLOPS[dt]
        for (M, N, K) in YARDSTICK_SHAPES:
            per = (M * K + K * N + M * N) * esz
            nrot = max(2, int(ring_mb * 1e6 // per) + 1)
            flop = 2.0 * M * N * K
            # the library
            As = [torch.randn(M, K, device=dev, dtype=tdt) for _ in range(nrot)]
            Bs = [torch.randn(K, N, device=dev, dtype=tdt) for _ in range(nrot)]
            Cs = [torch.empty(M, N, device=dev, dtype=tdt) for _ in range(nrot)]
            for i in range(3):
                torch.matmul(As[i % nrot], Bs[i % nrot], out=Cs[i % nrot])
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(30):
                torch.matmul(As[i % nrot], Bs[i % nrot], out=Cs[i % nrot])
            e1.record()
            torch.cuda.synchronize()
            lib_us = e0.elapsed_time(e1) / 30 * 1e3
            del As, Bs, Cs
            torch.cuda.empty_cache()
            # this executor: the same product as a `dot`, on its own stream
            x = L.Operand(L.ax(("batch", M), ("model", K)))
            w = L.Operand(L.ax(K, N))
            low = L.dot([x, w], dt)
            c = hip.Compiled(low.text, dt, low.lanes, hip.FAST)
            bufs = [[hip.DeviceBuffer(M * K * esz), hip.DeviceBuffer(K * N * esz), hip.DeviceBuffer(M * N * esz)]
                    for _ in range(nrot)]
            for bb in bufs:
                bb[0].zero()
                bb[1].zero()
            # the ring as one recorded sequence (no host launch cost), repeated
            lib = hip.lib()
            tables = [(ctypes.c_void_p * 3)(*[b_.ptr for b_ in bb]) for bb in bufs]
            bt = ctypes.c_void_p()
            hip.check(lib.presk_hip_batch_create(ctypes.byref(bt)))
            try:
                for t in tables:
                    hip.check(lib.presk_hip_batch_add(bt, c.handle, t, 0, max(c.split_bound, 0)))
                hip.check(lib.presk_hip_batch_graph_branches(bt, 1))
                for _ in range(2):
                    hip.check(lib.presk_hip_batch_run(bt, None))
                hip.sync()
                reps = 8
                t0 = time.perf_counter()
                for _ in range(reps):
                    hip.check(lib.presk_hip_batch_run(bt, None))
                hip.sync()
                own_us = (time.perf_counter() - t0) / (reps * nrot) * 1e6
            finally:
                lib.presk_hip_batch_release(bt)
            del bufs
            lt, ot = flop / lib_us / 1e6, flop / own_us / 1e6
            rows.append(f"| {M} x {N} x {K} | {dt} | {lib_us:.1f} | {lt:.1f} | {100 * lt / peak:.1f} | {own_us:.1f} | {ot:.1f} | "
                        f"{100 * ot / peak:.1f} | {c.order} |")
            print(f"[yardstick] {dt} {M}x{N}x{K}: library {lib_us:.1f} us, executor {own_us:.1f} us", file=sys.stderr, flush=True)
    with open(path, "w") as f:
        f.write("\n".join(rows) + "\n")


# the other configurations, timed after the headline (rows of the same line)
SUPPLEMENTARY = [("gpt-step", "bf16", None), ("gpt-forward", "f32", "@" + os.path.join(ROOT, "presk_amd", "realizations", "course_gpt_mixed.json")),
                 ("linear", "f32", None), ("mlp", "bf16", None), ("llama", "bf16", None)]


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
    ap.add_argument("--no-supplementary", action="store_true", help="time the headline workload only")
    ap.add_argument("--eager", action="store_true", help="issue the launches one by one instead of one HIP graph")
    ap.add_argument("--dominant-only", type=int, default=0, metavar="N",
                    help="after the timing pass, run the dominant launch alone N times and exit (for rocprofv3 --pmc)")
    ap.add_argument("--dominant-match", default=None, metavar="TEXT",
                    help="take the dominant launch among those whose key contains TEXT (counter runs distort "
                         "the timings the choice is made on)")
    ap.add_argument("--peaks", action="store_true",
                    help="measure the device's MFMA rate (bf16, f32) and a copy nest's HBM rate, print them and exit")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run a plain copy-like nest (neg over 64 Mi f32) 3 times and exit: the counters' calibration")
    ap.add_argument("--per-launch", default=None, metavar="FILE",
                    help="also time each distinct launch alone and write a markdown table of them to FILE")
    ap.add_argument("--yardstick", default=None, metavar="FILE",
                    help="time torch.matmul (the vendor library) beside this executor's contraction on the "
                         "configurations' GEMM shapes, write a markdown table to FILE and exit")
    ap.add_argument("--traffic-run", default=None, metavar="KEYS_JSON",
                    help="the counter runs' program: every distinct launch 3 times after a memset delimiter (run "
                         "under rocprofv3 --pmc), the launch keys written to KEYS_JSON; exits")
    ap.add_argument("--traffic-table", nargs=4, default=None, metavar=("KEYS_JSON", "FETCH_GLOB", "WRITE_GLOB", "OUT"),
                    help="profiles/traffic.json from the FETCH_SIZE and WRITE_SIZE runs of --traffic-run; exits")
    ap.add_argument("--cpu-rows", type=int, default=None)
    ap.add_argument("--cpu-child", nargs=3, type=int, default=None, metavar=("ROWS", "THREADS", "CORE"),
                    help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "the executor runs on one device, and sharding across GPUs is not built.", file=sys.stderr)
        sys.exit(2)
    dtype = args.dtype or ("bf16" if args.workload in ("mlp", "llama") else "f32")
    if args.traffic_table:
        traffic_table(*args.traffic_table)
        return
    if args.cpu_child:
        rows, th, core = args.cpu_child
        cpu_child(args.workload, dtype, rows, th, core, args.realize, args.dropout, args.adamw)
        return
    # the CPU baseline first, in child processes, before the GPU is touched
    cpu = None
    if not args.no_cpu and not args.copy_probe and not args.dominant_only and not args.yardstick and not args.traffic_run \
            and not args.peaks:
        # gpt-step: B 16 x T 256, the batch of the reference's own published rows
        rows_all = args.cpu_rows or {"mlp": 2048, "linear": 512, "gpt-step": 4096, "gpt-forward": 4096}.get(args.workload)
        rows_one = {"mlp": 256, "linear": 64, "gpt-step": 256, "gpt-forward": 256}.get(args.workload)
        if rows_all:
            cpu = cpu_baseline(args.workload, dtype, rows_all, rows_one, args.realize, args.dropout, args.adamw)

    from presk_amd import hip

    if args.copy_probe:
        copy_probe()
        return
    if args.yardstick:
        yardstick(args.yardstick)
        return
    if args.traffic_run:
        traffic_run(args.traffic_run)
        return
    if args.peaks:
        print(json.dumps({"measured_peaks": measured_peaks()}), flush=True)
        return
    # the measured peaks beside the vendor's (not in the counter runs of one launch)
    peaks = None if args.dominant_only else measured_peaks()
    rec, p, (ln, c) = measure(args.workload, dtype, args.steps, args.warmup, args.realize, args.dropout, args.adamw,
                              args.eager, args.dominant_match, peaks)
    if args.per_launch:
        per_launch_table(p, args.per_launch)
    if args.dominant_only:
        hip.sync()
        for _ in range(args.dominant_only):
            hip.check(hip.lib().presk_hip_run(c.handle, ln.table, 0, max(c.split_bound, 0), None))
        hip.sync()
        print(json.dumps({"dominant": launch_key(ln), "runs": args.dominant_only}), flush=True)
        return
    metric = {"gpt-step": METRIC, "gpt-forward": "tokens/sec course-GPT forward and loss (config 3)",
              "llama": "tokens/sec Llama-7B-shaped forward (config 5); matmul TFLOP/s as % of MFMA peak"}.get(
        args.workload, f"rows/sec {args.workload} (a supplementary workload)")
    out = {"metric": metric, "value": rec["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": rec["ms_per_step"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": rec["dtype"],
           "data": DATA.get(args.workload, "synthetic (seeded N(0,1) inputs, xavier weights)"),
           "config": rec["config"], "matmul_tflops": rec["matmul_tflops"], "matmul_frac_of_peak": rec["matmul_frac_of_peak"],
           "roofline": rec["roofline"], "kernels": rec["kernels"], "kernel_ms_sum": rec["kernel_ms_sum"]}
    if peaks:
        out["measured_peaks"] = peaks
    if cpu is not None:
        out["cpu_baseline"] = cpu
    del p
    if not args.no_supplementary and args.workload == "gpt-step" and not args.realize and not args.adamw and not args.eager:
        sup = []
        for name, dt, real in SUPPLEMENTARY:
            if (name, dt) == (args.workload, dtype):
                continue
            r, q, _ = measure(name, dt, 10 if name != "llama" else 5, 3 if name != "llama" else 2, real, peaks=peaks)
            del q
            gc.collect()
            sup.append({k: r[k] for k in ("value", "unit", "ms_per_step", "dtype", "config", "matmul_tflops",
                                          "matmul_frac_of_peak", "roofline")})
            print(f"[bench] {name} {dt}: {r['ms_per_step']} ms", file=sys.stderr, flush=True)
        out["supplementary"] = sup
    print(json.dumps(out), flush=True)


TRAFFIC = _traffic_table()

if __name__ == "__main__":
    main()
