"""GPU tests of the eviction-regime classifier (perfect_eviction: the logit
ceiling and classify_eviction, one oc_block_regimes launch), in the
scenarios of the reference's tests/test_perfect_eviction.py and on random
tables against the oracle's float32 restatement.

Bars: regimes and counts exact (random tables keep every gap at least 1e-3
away from the threshold); ceilings and gaps within 2e-6 relative of the
oracle (the query norm's float32 summation order is free)."""

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield


def _pe():
    from orthocache_gpu import perfect_eviction
    return perfect_eviction


def test_block_beta():
    q = torch.zeros(2, 3, 4)
    q[0, 0] = torch.tensor([3.0, 4.0, 0.0, 0.0])  # ||q|| = 5 for head 0
    q[1, 1] = torch.tensor([0.0, 0.0, 1.0, 0.0])
    e = torch.tensor([[16.0, 4.0, 9.0], [0.0, 1.0, 0.0]])
    beta = _pe().compute_block_beta(q.to(DEV), e.to(DEV), head_dim=4)
    assert torch.equal(beta.cpu(), torch.tensor([[10.0, 1.0, 0.0], [0.0, 0.5, 0.0]]))


def _scenario():
    torch.manual_seed(0)
    q = torch.randn(1, 1, 64)
    energies = torch.tensor([[100.0], [0.001], [50.0], [0.0001]])
    mask = torch.tensor([True, False, True, False])
    return q.to(DEV), energies.to(DEV), torch.tensor(100.0), mask.to(DEV)


def test_classification_is_exhaustive_and_retained_are_zero():
    q, e, z, m = _scenario()
    meta = _pe().classify_eviction(q, e, z, m, 64)
    assert meta.num_retained + meta.num_perfect + meta.num_statistical == 4
    assert meta.regime[0] == 0 and meta.regime[2] == 0
    assert meta.num_perfect == 2 and meta.regime[1] == 1 and meta.regime[3] == 1
    assert meta.underflow_threshold == _pe().FLOAT32_UNDERFLOW_THRESHOLD


def test_low_and_high_energy_regimes():
    pe = _pe()
    q = torch.ones(1, 1, 64, device=DEV) * 0.1
    meta = pe.classify_eviction(q, torch.tensor([[1e-10]], device=DEV), torch.tensor(100.0),
                                torch.tensor([False], device=DEV), 64)
    assert meta.num_perfect == 1 and meta.regime[0] == 1
    q = torch.ones(1, 1, 64, device=DEV) * 10.0
    meta = pe.classify_eviction(q, torch.tensor([[10000.0]], device=DEV), torch.tensor(15.0),
                                torch.tensor([False], device=DEV), 64)
    assert meta.num_statistical == 1 and meta.regime[0] == 2


def test_multi_head_and_per_head_masks():
    pe = _pe()
    torch.manual_seed(1)
    q = torch.randn(1, 4, 64, device=DEV)
    e = torch.rand(8, 4, device=DEV) * 0.001
    mask = torch.tensor([True, False] * 4, device=DEV)
    meta = pe.classify_eviction(q, e, torch.tensor(100.0), mask, 64)
    assert meta.num_retained == 4 and meta.num_perfect + meta.num_statistical == 4
    # a (blocks, heads) mask counts a block as retained when any head keeps it
    m2 = torch.zeros(8, 4, dtype=torch.bool, device=DEV)
    m2[0, 3] = True
    meta2 = pe.classify_eviction(q, e, torch.tensor([3.0, 100.0], device=DEV), m2, 64)
    assert meta2.num_retained == 1 and meta2.regime[0] == 0


@pytest.mark.parametrize("gap", [0.0, 44.36, 88.71, 88.72, 88.73, 100.0, 200.0])
def test_gap_classification(gap):
    pe = _pe()
    meta = pe.classify_eviction(torch.zeros(1, 1, 4, device=DEV), torch.tensor([[0.0]], device=DEV),
                                torch.tensor(gap), torch.tensor([False], device=DEV), 4)
    assert (meta.num_perfect == 1) == (np.float32(gap) >= np.float32(pe.FLOAT32_UNDERFLOW_THRESHOLD))
    assert meta.num_perfect + meta.num_statistical == 1


def test_bfloat16_accumulator_threshold():
    pe = _pe()
    # gap 87.5: perfect for a bfloat16 accumulator (87.34), statistical for float32 (88.72)
    args = (torch.zeros(1, 1, 4, device=DEV), torch.tensor([[0.0]], device=DEV), 87.5,
            torch.tensor([False], device=DEV), 4)
    assert pe.classify_eviction(*args, accumulator_dtype="bfloat16").num_perfect == 1
    assert pe.classify_eviction(*args).num_statistical == 1


def test_nan_gap_is_neither_regime():
    # a NaN energy makes the ceiling and the gap NaN: both compares fail, so the
    # block keeps regime 0 and is counted in neither regime (the reference's
    # masked assignment leaves it untouched)
    pe = _pe()
    e = torch.tensor([[float("nan")], [1.0]], device=DEV)
    meta = pe.classify_eviction(torch.ones(1, 1, 4, device=DEV), e, 200.0,
                                torch.tensor([False, False], device=DEV), 4)
    assert meta.regime.tolist() == [0, 1]
    assert (meta.num_perfect, meta.num_statistical, meta.num_retained) == (1, 0, 0)
    assert torch.isnan(meta.beta[0]) and torch.isnan(meta.logit_gap[0])


@pytest.mark.parametrize("nb,H,sq,per_head,zvec", [(37, 32, 1, False, False), (300, 8, 5, True, True),
                                                    (1, 1, 3, False, True), (2100, 4, 2, True, False),
                                                    (64, 70, 1, True, False)])
def test_random_tables_vs_oracle(nb, H, sq, per_head, zvec):
    pe = _pe()
    rng = np.random.default_rng(nb * 7 + H)
    d = 128
    q = rng.standard_normal((sq, H, d)).astype(np.float32)
    e = (rng.exponential(1.0, (nb, H)) * 10 ** rng.uniform(-6, 4, (nb, H))).astype(np.float32)
    e[rng.random((nb, H)) < 0.05] = -1e-3  # negative energies clamp to zero
    m = rng.random((nb, H) if per_head else (nb,)) < (0.1 if per_head else 0.4)
    z = (rng.uniform(20, 200, H) if zvec else np.float32(rng.uniform(50, 150))).astype(np.float32)
    reg, beta, gap, full, counts = O.block_regimes(q, e, d, z, m)
    # keep every evicted block's gap clear of the threshold
    near = np.abs(gap - np.float32(O.F32_UNDERFLOW)) < 1e-3
    m = (m.any(axis=1) | near)[:, None].repeat(H, 1) if per_head else (m | near)
    reg, beta, gap, full, counts = O.block_regimes(q, e, d, z, m)
    zt = torch.from_numpy(z).to(DEV) if zvec else float(z)
    meta = pe.classify_eviction(torch.from_numpy(q).to(DEV), torch.from_numpy(e).to(DEV), zt,
                                torch.from_numpy(m).to(DEV), d)
    assert np.array_equal(meta.regime.cpu().numpy(), reg)
    assert (meta.num_perfect, meta.num_statistical, meta.num_retained) == counts
    np.testing.assert_allclose(meta.beta.cpu().numpy(), beta, rtol=2e-6, atol=0)
    np.testing.assert_allclose(meta.logit_gap.cpu().numpy(), gap, rtol=2e-6, atol=1e-4)
    bf = pe.compute_block_beta(torch.from_numpy(q).to(DEV), torch.from_numpy(e).to(DEV), d)
    np.testing.assert_allclose(bf.cpu().numpy(), full, rtol=2e-6, atol=0)


def test_cpu_tensors_are_refused():
    with pytest.raises(RuntimeError, match="AMD GPU only"):
        _pe().classify_eviction(torch.zeros(1, 1, 4), torch.zeros(1, 1), 1.0, torch.tensor([False]), 4)
