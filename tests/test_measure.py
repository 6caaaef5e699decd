"""The gap of `presk solve`'s measurements (presk_amd/measure.py, after
crates/presk-driver/src/gap.rs:35-65): the largest absolute difference over
the leaves, a non-finite difference (an overflow, a NaN) counting as +inf
rather than being passed over."""
import math

import numpy as np

from presk_amd.measure import leaf_gap, leaf_max


def test_gap_is_the_largest_difference_over_leaves():
    ref = [np.array([1.0, -2.0, 3.0]), np.array([0.5])]
    got = [np.array([1.25, -2.0, 2.0]), np.array([0.5 + 2 ** -20])]
    assert leaf_gap(ref, got) == 1.0
    assert leaf_gap(ref, ref) == 0.0
    assert leaf_gap([np.zeros(0)], [np.zeros(0)]) == 0.0


def test_non_finite_differences_are_infinite():
    ref = [np.array([1.0, 2.0])]
    assert leaf_gap(ref, [np.array([1.0, np.nan])]) == math.inf
    assert leaf_gap(ref, [np.array([np.inf, 2.0])]) == math.inf
    assert leaf_gap(ref, [np.array([-np.inf, 2.0])]) == math.inf
    # f64::max passes over a NaN; the gap does not
    assert leaf_gap([np.array([np.nan, 0.0])], [np.array([np.nan, 0.0])]) == math.inf


def test_leaf_max():
    assert leaf_max([np.array([1.0, -3.0]), np.array([2.0])]) == 3.0
    assert leaf_max([np.array([1.0, np.nan])]) == math.inf
