"""CPU tests of the compact pipeline's host logic (perfect_eviction: the
logit ceiling, the regime classifier and the scalar check), in the
scenarios of the reference's tests/test_perfect_eviction.py."""

import math

import numpy as np
import pytest
import torch

from orthocache_gpu.perfect_eviction import (BFLOAT16_UNDERFLOW_THRESHOLD, FLOAT32_UNDERFLOW_THRESHOLD,
                                             classify_eviction, compute_block_beta, perfect_eviction_check)


def test_underflow_constants_are_the_float_limits():
    # e^-x is below the smallest float32 subnormal (2^-149) for x > 149 ln 2 ~ 103.28 and
    # below the smallest normal (2^-126) for x > 126 ln 2 ~ 87.34; 88.72 ~ ln(FLT_MAX)
    assert FLOAT32_UNDERFLOW_THRESHOLD == 88.72 and BFLOAT16_UNDERFLOW_THRESHOLD == 87.34
    assert np.float32(np.exp(np.float32(-FLOAT32_UNDERFLOW_THRESHOLD))) < np.finfo(np.float32).tiny
    assert abs(math.log(np.finfo(np.float32).max) - FLOAT32_UNDERFLOW_THRESHOLD) < 0.01


def test_block_beta():
    q = torch.zeros(2, 3, 4)
    q[0, 0] = torch.tensor([3.0, 4.0, 0.0, 0.0])  # ||q|| = 5 for head 0
    q[1, 1] = torch.tensor([0.0, 0.0, 1.0, 0.0])
    e = torch.tensor([[16.0, 4.0, 9.0], [0.0, 1.0, 0.0]])
    beta = compute_block_beta(q, e, head_dim=4)
    assert torch.allclose(beta, torch.tensor([[10.0, 1.0, 0.0], [0.0, 0.5, 0.0]]))


def test_check_boundary_and_dtypes():
    assert perfect_eviction_check(100.0, 11.28) and perfect_eviction_check(88.72, 0.0)
    assert not perfect_eviction_check(88.71, 0.0)
    assert perfect_eviction_check(87.5, 0.0, "bfloat16") and not perfect_eviction_check(87.5, 0.0)


def _scenario():
    torch.manual_seed(0)
    q = torch.randn(1, 1, 64)
    energies = torch.tensor([[100.0], [0.001], [50.0], [0.0001]])
    mask = torch.tensor([True, False, True, False])
    return q, energies, torch.tensor(100.0), mask


def test_classification_is_exhaustive_and_retained_are_zero():
    q, e, z, m = _scenario()
    meta = classify_eviction(q, e, z, m, 64)
    assert meta.num_retained + meta.num_perfect + meta.num_statistical == 4
    assert meta.regime[0] == 0 and meta.regime[2] == 0
    assert meta.num_perfect == 2 and meta.regime[1] == 1 and meta.regime[3] == 1
    assert meta.underflow_threshold == FLOAT32_UNDERFLOW_THRESHOLD


def test_low_and_high_energy_regimes():
    q = torch.ones(1, 1, 64) * 0.1
    meta = classify_eviction(q, torch.tensor([[1e-10]]), torch.tensor(100.0), torch.tensor([False]), 64)
    assert meta.num_perfect == 1 and meta.regime[0] == 1
    q = torch.ones(1, 1, 64) * 10.0
    meta = classify_eviction(q, torch.tensor([[10000.0]]), torch.tensor(15.0), torch.tensor([False]), 64)
    assert meta.num_statistical == 1 and meta.regime[0] == 2


def test_multi_head_and_per_head_masks():
    torch.manual_seed(1)
    q = torch.randn(1, 4, 64)
    e = torch.rand(8, 4) * 0.001
    mask = torch.tensor([True, False] * 4)
    meta = classify_eviction(q, e, torch.tensor(100.0), mask, 64)
    assert meta.num_retained == 4 and meta.num_perfect + meta.num_statistical == 4
    # a (blocks, heads) mask counts a block as retained when any head keeps it
    m2 = torch.zeros(8, 4, dtype=torch.bool)
    m2[0, 3] = True
    meta2 = classify_eviction(q, e, torch.tensor([3.0, 100.0]), m2, 64)
    assert meta2.num_retained == 1 and meta2.regime[0] == 0


@pytest.mark.parametrize("gap", [0.0, 44.36, 88.71, 88.72, 88.73, 100.0, 200.0])
def test_gap_classification(gap):
    meta = classify_eviction(torch.zeros(1, 1, 4), torch.tensor([[0.0]]), torch.tensor(gap), torch.tensor([False]), 4)
    assert (meta.num_perfect == 1) == (np.float32(gap) >= np.float32(FLOAT32_UNDERFLOW_THRESHOLD))
    assert meta.num_perfect + meta.num_statistical == 1
