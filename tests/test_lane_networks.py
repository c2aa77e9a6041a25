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
3. flat_map_lpt (csrc/oc_kernels.h): the same for the long-shares-first
   layout, whose share count must also stay within flat_lpt_slots (the grid
   and partial slots the host allocates) and its per-row count within the
   merge's bound.
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


def _flat_lpt_slots(w, rows, pct, div):
    """flat_lpt_slots (csrc/oc_kernels.h): the slot bound the host allocates"""
    return w * pct // 100 + (w * (100 - pct) * div + 99) // 100 + rows * (div + 1) + 1


def _flat_lpt_map(lens, tiles_max, target, qcap, pct, div, kdt=256, mistake=None):
    """flat_map_lpt (csrc/oc_kernels.h) restated: for every blockIdx below the
    share count, (row, share index, row's share count, row's first slot, b0,
    b1), with pass 3's scan done chunk by chunk of kdt rows as the kernel does."""
    n = [(min(max(l, 0), tiles_max * 64) + 63) // 64 for l in lens]
    total, nmax = sum(n), max(n)
    f100 = pct + (100 - pct) * div
    ucap = -(-nmax * f100 // (100 * (qcap - div - 1)))
    u = max(1, -(-total // target), ucap)
    v = -(-u // div)

    def cut(x):
        nb = x * pct // (100 * u)
        ns = 1 if x == 0 else -(-(x - nb * u) // v)
        return nb, ns

    big = sum(cut(x)[0] for x in n)
    out = {}
    cb = cs = ca = 0
    for c in range(0, len(n), kdt):
        chunk = [cut(x) for x in n[c:c + kdt]]
        ib = np.cumsum([b for b, _ in chunk])
        is_ = np.cumsum([s for _, s in chunk])
        ia = np.cumsum([b + s for b, s in chunk])
        for j, (nb, ns) in enumerate(chunk):
            r = c + j
            fb = cb + int(ib[j]) - nb
            fs = (0 if mistake == "short_after_long" else big) + cs + int(is_[j]) - ns
            slot0 = ca + int(ia[j]) - nb - ns
            for g in range(nb):
                out.setdefault(fb + g, []).append((r, g, nb + ns, slot0, g * u, (g + 1) * u))
            L = n[r] - nb * u
            for h in range(ns):
                out.setdefault(fs + h, []).append((r, nb + h, nb + ns, slot0, nb * u + L * h // ns,
                                                   nb * u + L * (h + 1) // ns))
        cb += int(ib[-1])
        cs += int(is_[-1])
        ca += int(ia[-1])
    return n, out, big


def _flat_lpt_check(lens, t_max, target, qcap, pct, div, mistake=None, kdt=256):
    n, out, big = _flat_lpt_map(lens, t_max, target, qcap, pct, div, kdt=kdt, mistake=mistake)
    count = len(out)
    assert all(len(v) == 1 for v in out.values())                # one share per slot
    assert sorted(out) == list(range(count))                       # slots 0 .. count-1 all used
    assert count <= _flat_lpt_slots(target, len(lens), pct, div)   # the grid the host launches
    cover = {r: [] for r in range(len(n))}
    slots = set()
    for bid in range(count):
        r, g, q, slot0, b0, b1 = out[bid][0]
        assert q <= qcap                                          # the merge's LDS bound
        assert 0 <= g < q and (slot0 + g) not in slots
        slots.add(slot0 + g)
        cover[r].append((g, b0, b1))
    assert max(slots) < _flat_lpt_slots(target, len(lens), pct, div)
    for r in range(len(n)):
        parts = sorted(cover[r])
        assert [g for g, _, _ in parts] == list(range(len(parts)))
        tiles = [t for _, b0, b1 in parts for t in range(b0, b1)]
        assert tiles == list(range(n[r]))                          # the shares tile the row in order
    # long shares (U tiles) are numbered before every short one
    longs = [out[b][0][5] - out[b][0][4] for b in range(big)]
    assert len(set(longs)) <= 1


def test_flat_lpt_layout_tiles_every_row_once():
    rng = np.random.default_rng(2)
    for _ in range(200):
        rows = int(rng.integers(1, 700))
        t_max = int(rng.integers(1, 3000))
        lens = [int(rng.choice([0, rng.integers(0, t_max * 64 + 1), t_max * 64, rng.integers(0, 200)]))
                for _ in range(rows)]
        target, qcap = int(rng.choice([256, 512, 1024, 2048])), int(rng.choice([256, 512]))
        pct, div = int(rng.choice([0, 50, 75, 90, 95, 100])), int(rng.choice([1, 2, 4, 8, 16]))
        _flat_lpt_check(lens, t_max, target, qcap, pct, div)


def test_flat_lpt_layout_planted_mistake():
    # numbering the short shares from 0 (forgetting the long shares before
    # them) puts two shares on one slot
    lens = [64 * 700, 64 * 300, 64 * 50]
    _flat_lpt_check(lens, 700, 64, 512, 75, 4)
    with pytest.raises(AssertionError):
        _flat_lpt_check(lens, 700, 64, 512, 75, 4, mistake="short_after_long")


def test_flat_lpt_layout_many_rows():
    # more rows than the kernel's 4-wave (1024) or 8-wave (2048) workgroups
    # keep in registers, scanned chunk by chunk; most rows get one short share
    rng = np.random.default_rng(3)
    lens = [int(v) for v in rng.integers(0, 257, size=2100)]
    lens[:40:3] = [0] * len(lens[:40:3])
    for kdt in (256, 512):
        for qcap in (256, 512):
            _flat_lpt_check(lens, 4, 1024, qcap, 90, 4, kdt=kdt)
