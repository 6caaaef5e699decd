"""The graph-branch planner (presk_amd/csrc/branches.hpp: each step's read
and written byte spans, the streams and the waits of a branched capture) on
whole recorded launch sequences, on the CPU under AddressSanitizer and
UndefinedBehaviorSanitizer -- every index into a pointer table, the per-stream
tables and the waits checked by the sanitizers -- and its plan checked for
order: for 2, 4 and 8 branches, every pair of steps that conflict (one
writes bytes the other reads or writes, or both launch one compiled kernel)
is ordered by the streams' program order and the waits.

The sequences are built as Program.prepare and Program.record hand them to
the executor (host inputs declared as configs.load_inputs declares them,
conversions at the edges, outputs, stacked leaves inside their parents,
dropout masks first), at addresses laid out as Buffers allocates them; the
driver (tests/native/branch_plan.cpp) checks each pointer table's length
against the one presk_hip_batch_add copies for its kernel."""
import os
import shutil
import subprocess

import pytest

from presk_amd import configs, gpt, hip, llama
from presk_amd.program import INTS, nbytes, numel
from presk_amd.realize import Realization

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "presk_amd", "csrc")
CODES = {"f64": 0, "f32": 1, "bf16": 2, "f16": 4, "e8m15": 5}

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("plan") / "branch_plan")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-I", CSRC, os.path.join(ROOT, "tests", "native", "branch_plan.cpp"),
           os.path.join(CSRC, "ir.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def sequence(p) -> str:
    addr, meta = {}, {}
    top = [1 << 32]

    def alloc(name, ty, count):
        if name in addr:
            return addr[name]
        if name in p.bufs.views:
            parent, first, pty, pcount = p.bufs.views[name]
            base = alloc(parent, pty, pcount)
            addr[name], meta[name] = base + nbytes(ty, first), (ty, count)
            return addr[name]
        addr[name], meta[name] = top[0], (ty, count)
        top[0] += (max(nbytes(ty, count), 1) + 255) // 256 * 256
        return addr[name]

    produced = {ln.out for ln in p.launches}
    for ln in p.launches:
        for name, (ty, count) in zip(ln.ins, configs._input_specs(ln.low)):
            if name not in produced:
                alloc(name, p.input_types.get(name, ty) if ty != "i64" else ty, max(count, 1))
    flag = alloc("#flag", "i64", 1)
    keys = alloc("#keys", "i64", 4 * max(len(p.keys), 1))
    lines, kid = [], {}
    for name, slot, rate, ty, count in p.masks:
        alloc(name, ty, count)
        lines.append(f"S D {keys + 32 * slot} {addr[name]} {CODES[ty]} {count} {rate!r}")
    converted = {}
    for ln in p.launches:
        names = []
        for n in ln.ins:
            src_ty, count = meta[n]
            if src_ty not in ("i64", ln.low.dtype) + INTS:
                key = (n, ln.low.dtype)
                if key not in converted:
                    dst = f"{n}@{ln.low.dtype}"
                    alloc(dst, ln.low.dtype, count)
                    lines.append(f"S C {addr[n]} {addr[dst]} {flag} {CODES[src_ty]} {CODES[ln.low.dtype]} {count}")
                    converted[key] = dst
                n = converted[key]
            names.append(n)
        alloc(ln.out, ln.low.dtype if ln.low.out_kind == "real" else "i64", numel(ln.low.out_axes))
        ptrs = [addr[n] for n in names] + [addr[ln.out]] + [addr[s] for s in ln.scales]
        if ln.low.dtype in ("f16", "e8m15") and ln.low.out_kind == "real":
            ptrs.append(flag)
        key = (ln.low.text, ln.low.dtype, ln.low.lanes)
        if key not in kid:
            kid[key] = len(kid)
            text = ln.low.text.encode()
            lines.append(f"K {kid[key]} {ln.low.dtype} {ln.low.lanes} {len(text)}\n{ln.low.text}")
        lines.append(f"S L {kid[key]} {len(ptrs)} " + " ".join(str(x) for x in ptrs))
    return "\n".join(lines) + "\n"


PROGRAMS = {
    # the headline's sequence: config 4 at full size, f32 (the case whose
    # branched capture faulted, at TINY size on the device)
    "course-f32": lambda: gpt.build(gpt.COURSE, "f32", mode=hip.FAST)[0],
    "course-bf16": lambda: gpt.build(gpt.COURSE, "bf16", mode=hip.FAST)[0],
    # conversions at the edges and dropout masks
    "tiny-mixed-dropout": lambda: gpt.build(gpt.TINY, "f32", mode=hip.EXACT, dropout=0.2, realize=Realization.of_json(
        {"default": "bf16", "order": {"kind": "sequential"}, "params": {"blocks.attn.wq.w": "f16"}}))[0],
    "llama-bf16": lambda: llama.build(llama.LLAMA_7B, "bf16", mode=hip.FAST)[0],
}


@pytest.mark.parametrize("name", list(PROGRAMS))
def test_branch_plan_under_sanitizers(driver, tmp_path, name):
    p = PROGRAMS[name]()
    f = tmp_path / "seq.txt"
    f.write_text(sequence(p))
    r = subprocess.run([driver, str(f)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and r.stdout.endswith("OK\n"), (r.stdout[-2000:], r.stderr[-6000:])
    print(r.stdout)


def test_the_order_check_finds_a_missing_wait(driver, tmp_path):
    """The checker itself: a plan of the course step that loses one of its
    waits (each orders a step after a step it depends on) must be found."""
    f = tmp_path / "seq.txt"
    f.write_text(sequence(PROGRAMS["course-f32"]()))
    r = subprocess.run([driver, str(f), "--drop-wait"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and r.stdout.count(": found") == 3, (r.stdout[-2000:], r.stderr[-4000:])
