"""CPU restatements of two lane-level algorithms of the decode kernel,
checked against what the mathematics fixes (no GPU needed).

1. tile_energies_mfma (csrc/oc_kernels.h): the band energies of a 64-token
   tile held in the matrix-core K layout (lane 16*kg + x holds tokens
   16*tb + x, columns 32*dc + 8*kg .. +8), with E_low formed by a DPP network
   (row_ror:8 add, then butterflies over quad_perm ^1, quad_perm ^2 and
   row_ror:4 with per-lane signs, DC lane dropped).  Must equal
   sum_{i in [1,8)} ||(W64 K)_i||^2 and sum_{i in [32,64)} ||(W64 K)_i||^2
   (fwht_fused_prototype.py:42-80) for either rotation direction.
2. flat_map (csrc/oc_kernels.h): rows of different lengths get
   max(1, ceil(n_r / U)) workgroups; every slot below the total must map to
   exactly one (row, share) and the shares must tile each row.
"""

import numpy as np
import pytest

from oracle import orthocache_oracle as O


def _dpp_row(y, src):
    """y[lane] <- y[16 * (lane // 16) + src(lane % 16)] (a DPP row permutation)"""
    lanes = np.arange(64)
    return y[16 * (lanes // 16) + np.array([src(i % 16) for i in lanes])]


def _energies_lane_network(k, ror_right, mistake=None):
    d = k.shape[1]
    vals = np.zeros((64, 4, d // 4))
    for lane in range(64):
        kg, x = lane >> 4, lane & 15
        for tb in range(4):
            for dc in range(d // 32):
                vals[lane, tb, 8 * dc:8 * dc + 8] = k[16 * tb + x, 32 * dc + 8 * kg:32 * dc + 8 * kg + 8]
    ror = (lambda n: (lambda i: (i - n) & 15)) if ror_right else (lambda n: (lambda i: (i + n) & 15))
    x = (np.arange(64) & 15)[:, None]
    s0, s1, s2 = (np.where(x & b, -1.0, 1.0) for b in (1, 2, 4))
    low_lane = ((x & 7) != 0) & (x < 8)
    f = vals
    if mistake == "swap_pairs":
        e_high = 0.5 * (((f[:, 0] - f[:, 1]) ** 2) + ((f[:, 2] - f[:, 3]) ** 2)).sum()
    else:
        e_high = 0.5 * (((f[:, 0] - f[:, 2]) ** 2) + ((f[:, 1] - f[:, 3]) ** 2)).sum()
    y = (f[:, 0] + f[:, 1]) + (f[:, 2] + f[:, 3])
    if mistake != "no_ror8":
        y = y + _dpp_row(y, ror(8))
    y = _dpp_row(y, lambda i: i ^ 1) * s0 + y
    y = _dpp_row(y, lambda i: i ^ 2) * s1 + y
    if mistake != "no_ror4":
        y = _dpp_row(y, ror(4)) * s2 + y
    if mistake == "keep_dc":
        low_lane = x < 8
    e_low = np.where(low_lane, y * y, 0.0).sum() / 64.0
    return e_low, e_high


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("kind", ["noise", "dc_offset", "smooth", "integer"])
def test_mfma_layout_energy_network(d, kind):
    rng = np.random.default_rng(d + len(kind))
    w = O.walsh_matrix().astype(np.float64)
    if kind == "smooth":
        c = np.zeros((64, d))
        c[1:5] = rng.standard_normal((4, d))
        k = w @ c
    elif kind == "integer":
        k = rng.integers(-4, 5, size=(64, d)).astype(np.float64)
    else:
        k = rng.standard_normal((64, d)) + (7.0 if kind == "dc_offset" else 0.0)
    x = w @ k
    want_low, want_high = (x[1:8] ** 2).sum(), (x[32:64] ** 2).sum()
    for ror_right in (False, True):
        e_low, e_high = _energies_lane_network(k, ror_right)
        np.testing.assert_allclose(e_low, want_low, rtol=1e-10, atol=1e-9)
        np.testing.assert_allclose(e_high, want_high, rtol=1e-10, atol=1e-9)


@pytest.mark.parametrize("mistake", ["no_ror4", "no_ror8", "keep_dc", "swap_pairs"])
def test_energy_network_catches_planted_mistakes(mistake):
    """Each plausible slip in the network (a dropped stage, the DC lane kept,
    E_high pairs (tb, tb+1) instead of (tb, tb+2)) changes the result."""
    rng = np.random.default_rng(0)
    k = rng.standard_normal((64, 128)) + 3.0
    x = O.walsh_matrix().astype(np.float64) @ k
    e_low, e_high = _energies_lane_network(k, False, mistake=mistake)
    ok_low = np.isclose(e_low, (x[1:8] ** 2).sum(), rtol=1e-6)
    ok_high = np.isclose(e_high, (x[32:64] ** 2).sum(), rtol=1e-6)
    assert not (ok_low and ok_high)


def _flat_table(lens, tiles_max, target, qcap):
    n = [(min(max(l, 0), tiles_max * 64) + 63) // 64 for l in lens]
    total, nmax = sum(n), max(n)
    u = max(1, -(-total // target), -(-nmax // qcap))
    return n, [max(1, -(-x // u)) for x in n]


def test_flat_layout_covers_every_slot_once():
    rng = np.random.default_rng(1)
    for _ in range(300):
        rows = int(rng.integers(1, 700))
        t_max = int(rng.integers(1, 3000))
        lens = [int(rng.choice([0, rng.integers(0, t_max * 64 + 1), t_max * 64, rng.integers(0, 200)]))
                for _ in range(rows)]
        target, qcap = int(rng.choice([512, 1024, 2048])), int(rng.choice([256, 512]))
        n, q = _flat_table(lens, t_max, target, qcap)
        assert sum(q) <= target + rows          # the slots the host allocates
        assert max(q) <= qcap                   # the merge's LDS bound
        owner = {}
        first = 0
        for r, qr in enumerate(q):              # the kernel's chunked scan gives the same prefix
            for b in range(first, first + qr):
                assert b not in owner
                owner[b] = (r, b - first)
            first += qr
        assert sorted(owner) == list(range(sum(q)))
        for r in range(rows):
            cover = []
            for g in range(q[r]):
                cover += range(n[r] * g // q[r], n[r] * (g + 1) // q[r])
            assert cover == list(range(n[r]))
