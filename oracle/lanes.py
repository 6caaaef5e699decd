"""oracle/lanes.py -- TEST INFRASTRUCTURE ONLY (the parity oracle).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything under oracle/.  Never the product path.

The executor's own declared order for FAST mode's row sums, `lanes64xV-tree`
(an order of this executor's, like its `rows-in-chunks(64)`; the reference's
`ReductionOrder` has no such member, crates/presk-rt/src/lib.rs:251-285):
a row of n elements is cut into blocks of V consecutive elements, block b
belonging to lane b mod 64 of 64; each lane adds its elements in increasing
index from +0 in f32; the 64 lane sums are then added by a balanced pairwise
tree over the lane index, ((s0 + s1) + (s2 + s3)) + ..., in f32.  numpy's
float32 arithmetic rounds each operation once, as the device's does.
"""
from __future__ import annotations

import numpy as np


def lanes_tree_sum(x: np.ndarray, vec: int) -> np.ndarray:
    """The sum of each row of `x` ([rows, n], float32) in the lanes64 tree
    order with blocks of `vec` elements; float32 [rows]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    nb = (n + vec - 1) // vec
    ch = (nb + 63) // 64
    s = np.zeros((rows, 64), np.float32)
    lanes = np.arange(64)
    for j in range(ch):
        for i in range(vec):
            e = (j * 64 + lanes) * vec + i
            ok = e < n
            v = np.zeros((rows, 64), np.float32)
            v[:, ok] = x[:, e[ok]]
            s = s + v
    for d in (1, 2, 4, 8, 16, 32):
        s = s + s[:, lanes ^ d]
    return s[:, 0].copy()
