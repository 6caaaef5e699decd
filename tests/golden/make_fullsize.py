"""Writes tests/golden/fullsize_c4.json: digests of the oracle's run of
config 4 (the course-GPT training step at B 64 x T 256, the reference's
V 65, D 384, H 6, L 6) on gpt.host_inputs' seeded inputs, in f32 and bf16
storage -- sha256 of the loss's, the logits' and every parameter gradient's
storage bytes, and the loss's value.

The device's EXACT mode must reproduce these bytes at full size
(tests/test_gpu_fullsize.py), which carries the oracle's bit parity from the
TINY programs to the shapes bench.py times, where the oracle itself takes
minutes.  Run in this container (about ten minutes a storage type on eight
threads):

    python tests/golden/make_fullsize.py
"""
import hashlib
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def digests(env, names) -> dict:
    import numpy as np
    out = {"loss": hashlib.sha256(np.ascontiguousarray(env[names["loss"]]).tobytes()).hexdigest(),
           "logits": hashlib.sha256(np.ascontiguousarray(env[names["logits"]]).tobytes()).hexdigest()}
    for leaf, buf in sorted(names["grads"].items()):
        out["d." + leaf] = hashlib.sha256(np.ascontiguousarray(env[buf]).tobytes()).hexdigest()
    return out


def main():
    from presk_amd import gpt, hip
    from tests import cpu_program, fmt
    path = os.path.join(HERE, "fullsize_c4.json")
    table = json.load(open(path)) if os.path.exists(path) else {}
    s = gpt.COURSE
    host = gpt.host_inputs(s)
    for dt in sys.argv[1:] or ["f32", "bf16"]:
        t0 = time.time()
        p, _, names = gpt.build(s, dt, train=True, mode=hip.EXACT)
        env = cpu_program.run(p, host, threads=min(16, os.cpu_count() or 1), native=True)
        table[dt] = {"loss_value": float(fmt.decode(env[names["loss"]], dt)[0]), "sha256": digests(env, names),
                     "shape": {"V": s.V, "D": s.D, "H": s.H, "L": s.L, "B": s.B, "T": s.T}, "seed": 2}
        del env
        print(f"{dt}: {time.time() - t0:.0f} s, loss {table[dt]['loss_value']}", flush=True)
        with open(path, "w") as f:
            json.dump(table, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
