"""CPU tests of the compact pipeline's host logic: the underflow constants
and the scalar perfect-eviction check (perfect_eviction), in the scenarios
of the reference's tests/test_perfect_eviction.py.  The block classifier
itself runs on the GPU (tests/test_gpu_regimes.py); its oracle is pinned
here on hand-worked cases."""

import math

import numpy as np

from oracle import orthocache_oracle as O
from orthocache_gpu.perfect_eviction import (BFLOAT16_UNDERFLOW_THRESHOLD, FLOAT32_UNDERFLOW_THRESHOLD,
                                             perfect_eviction_check)


def test_underflow_constants_are_the_float_limits():
    # e^-x is below the smallest float32 subnormal (2^-149) for x > 149 ln 2 ~ 103.28 and
    # below the smallest normal (2^-126) for x > 126 ln 2 ~ 87.34; 88.72 ~ ln(FLT_MAX)
    assert FLOAT32_UNDERFLOW_THRESHOLD == 88.72 and BFLOAT16_UNDERFLOW_THRESHOLD == 87.34
    assert np.float32(np.exp(np.float32(-FLOAT32_UNDERFLOW_THRESHOLD))) < np.finfo(np.float32).tiny
    assert abs(math.log(np.finfo(np.float32).max) - FLOAT32_UNDERFLOW_THRESHOLD) < 0.01


def test_check_boundary_and_dtypes():
    assert perfect_eviction_check(100.0, 11.28) and perfect_eviction_check(88.72, 0.0)
    assert not perfect_eviction_check(88.71, 0.0)
    assert perfect_eviction_check(87.5, 0.0, "bfloat16") and not perfect_eviction_check(87.5, 0.0)
    # an unknown accumulator name falls back to the float32 margin
    assert not perfect_eviction_check(87.5, 0.0, "float16")


def test_oracle_regimes_hand_worked():
    # head norms 5 and 1 (max over the two query rows), energies 16 / 4 / 1,
    # d = 4: ceilings 5*4/2 = 10, 1*2/2 = 1, max(5*1/2, 0) = 2.5
    q = np.zeros((2, 2, 4), np.float32)
    q[0, 0, :2] = [3.0, 4.0]
    q[1, 1, 2] = 1.0
    e = np.array([[16.0, 0.0], [0.0, 4.0], [1.0, -2.0]], np.float32)
    reg, beta, gap, full, counts = O.block_regimes(q, e, 4, 100.0, np.array([False, False, True]))
    assert full.tolist() == [[10.0, 0.0], [0.0, 1.0], [2.5, 0.0]]
    assert beta.tolist() == [10.0, 1.0, 2.5]
    assert gap.tolist() == [90.0, 99.0, 97.5]
    assert reg.tolist() == [1, 1, 0] and counts == (2, 0, 1)
    # a gap of 88.71 is statistical, an array z uses its largest element
    reg, _, gap, _, counts = O.block_regimes(q, e, 4, np.array([1.0, 98.71], np.float32),
                                             np.array([False, True, True]))
    assert np.isclose(gap[0], 88.71, atol=1e-4) and reg.tolist() == [2, 0, 0] and counts == (0, 1, 2)
    # a (block, head) mask retains a block when any head keeps it
    m = np.array([[False, True], [False, False], [False, False]])
    reg, *_, counts = O.block_regimes(q, e, 4, 100.0, m)
    assert reg.tolist() == [0, 1, 1] and counts == (2, 0, 1)
