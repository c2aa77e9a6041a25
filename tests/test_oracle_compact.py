"""Pins of the oracle's compact-pipeline functions (CPU only): the 512-point
transform against the Sylvester matrix, band energies against closed forms
and Parseval, the query-aware bound against every logit of its block,
stream compaction against torch.argsort, and the pipeline's gates at their
extremes."""

import math

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O


def _h512():
    i = np.arange(512)
    pc = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2, -1.0, 1.0) / math.sqrt(512)


def test_fwht512_is_sylvester_and_involution():
    x = np.random.default_rng(0).standard_normal((512, 5))
    np.testing.assert_allclose(O.fwht512(x), _h512() @ x, atol=1e-12)
    np.testing.assert_allclose(O.fwht512(O.fwht512(x)), x, atol=1e-12)


def test_band_closed_forms_and_parseval():
    rng = np.random.default_rng(1)
    k = rng.standard_normal((1024, 2, 16))
    s = O.block_spectra(k)
    for b in range(2):
        for h in range(2):
            blk = k[512 * b:512 * (b + 1), h]
            np.testing.assert_allclose(s["e_high"][b, h], 0.5 * np.sum((blk[:256] - blk[256:]) ** 2), rtol=1e-12)
            total = s["e_low"][b, h] + s["e_mid"][b, h] + s["e_high"][b, h]
            dc2 = np.sum((blk.sum(axis=0) / math.sqrt(512)) ** 2)
            np.testing.assert_allclose(total + dc2, np.sum(blk ** 2), rtol=1e-12)
            np.testing.assert_allclose(s["e_ac"][b, h], total, rtol=1e-12)
            np.testing.assert_allclose(s["block_mean"][b, h], blk.mean(axis=0), atol=1e-14)
            # low band: the 64-point transform of the sum of the eight 64-token chunks
            ssum = blk.reshape(8, 64, 16).sum(axis=0)
            np.testing.assert_allclose(s["e_low"][b, h] + dc2, np.sum(ssum ** 2) / 8, rtol=1e-12)
    const = np.ones((512, 1, 4))
    c = O.block_spectra(const)
    assert c["e_low"][0, 0] < 1e-20 and c["e_mid"][0, 0] < 1e-20 and c["e_high"][0, 0] < 1e-20


def test_bound_dominates_every_logit():
    rng = np.random.default_rng(2)
    k = rng.standard_normal((1024, 3, 32)) + 0.3
    q = rng.standard_normal((4, 3, 32))
    s = O.block_spectra(k, q)
    for b in range(2):
        for h in range(3):
            lg = q[:, h] @ k[512 * b:512 * (b + 1), h].T / math.sqrt(32)
            assert (lg.max(axis=1) <= s["bounds"][:, b, h] + 1e-12).all()
    np.testing.assert_allclose(s["max_bound"], s["bounds"].max(axis=0))


def test_stream_compact_matches_argsort():
    rng = np.random.default_rng(3)
    for n in (1, 7, 300):
        m = rng.random(n) < 0.4
        idx, cnt = O.stream_compact(m)
        iota = torch.arange(n)
        want = torch.argsort(torch.where(torch.from_numpy(m), iota, n + iota), stable=True)
        assert np.array_equal(idx, want.numpy()) and cnt == int(m.sum())


def test_compact_forward_gates():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 2, 16))
    k = rng.standard_normal((1024, 2, 16))
    v = rng.standard_normal((1024, 2, 16))
    out, info = O.compact_forward(q, k, v, zeta_max=1e30, tau=-1e30)
    assert info["retained"] == 2
    dense = np.stack([O.dense_decode(q[:, h], np.repeat(k[None, :, h], 2, 0), np.repeat(v[None, :, h], 2, 0))
                      for h in range(2)], axis=1)
    np.testing.assert_allclose(out, dense, atol=1e-12)
    out0, info0 = O.compact_forward(q, k, v, zeta_max=-1.0, tau=-1e30)
    assert info0["retained"] == 0 and not out0.any() and info0["perfect"] + info0["statistical"] == 2
    mb = info["spectra"]["max_bound"]
    assert info["tau"] == -1e30
    _, auto = O.compact_forward(q, k, v)
    np.testing.assert_allclose(auto["tau"], mb.mean() - mb.std(ddof=1))
