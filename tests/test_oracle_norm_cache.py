"""Pins of the oracle's score-cache and decode-gate functions (CPU only):
closed forms, least squares, explicit loops and planted mistakes."""

import numpy as np
import pytest

from oracle import orthocache_oracle as O


def _tile(kind, d, seed):
    rng = np.random.default_rng(seed)
    if kind == "integer":
        return rng.integers(-4, 5, size=(64, d)).astype(np.float32)
    if kind == "dc":
        return (rng.standard_normal((64, d)) + 5.0).astype(np.float32)
    return rng.standard_normal((64, d)).astype(np.float32)


@pytest.mark.parametrize("kind", ["integer", "gauss", "dc"])
@pytest.mark.parametrize("d", [64, 128])
def test_band_norm_closed_forms(kind, d):
    k = _tile(kind, d, d)
    kd = k.astype(np.float64)
    high32 = np.sqrt(0.5 * np.sum((kd[:32] - kd[32:]) ** 2))
    g = kd[0:16] - kd[16:32] - kd[32:48] + kd[48:64]
    high48 = np.sqrt(0.25 * np.sum(g ** 2))
    if kind == "integer":
        # every partial sum is an exact small multiple of 1/64 in float32
        assert O.band_norm(k, 32, 64) == np.float32(high32)
        assert O.band_norm(k, 48, 64) == np.float32(high48)
    else:
        np.testing.assert_allclose(O.band_norm(k, 32, 64), high32, rtol=2e-6)
        np.testing.assert_allclose(O.band_norm(k, 48, 64), high48, rtol=2e-6)
    # the whole spectrum is the tile's Frobenius norm (Parseval)
    np.testing.assert_allclose(O.band_norm(k, 0, 64), np.linalg.norm(kd), rtol=2e-6)


def test_band_norm_planted_off_by_one_fails():
    k = _tile("gauss", 128, 3)
    kd = k.astype(np.float64)
    g = kd[0:16] - kd[16:32] - kd[32:48] + kd[48:64]
    assert not np.isclose(O.band_norm(k, 47, 64), np.sqrt(0.25 * np.sum(g ** 2)), rtol=1e-4)
    assert not np.isclose(O.band_norm(k, 48, 63), np.sqrt(0.25 * np.sum(g ** 2)), rtol=1e-4)


def test_band_norm_clamp_and_batch():
    z = np.zeros((64, 64), np.float32)
    z[:, 0] = 1e-30  # constant along tokens: all energy in the DC row
    assert O.band_norm(z, 48, 64) == 0.0
    keys = np.stack([np.concatenate([_tile("gauss", 64, s) for s in range(3)]) for _ in range(2)])
    got = O.band_norms(keys, 48, 64)
    assert got.shape == (2, 3)
    for r in range(2):
        for t in range(3):
            assert got[r, t] == O.band_norm(keys[r, 64 * t:64 * t + 64], 48, 64)


@pytest.mark.parametrize("d,low_band", [(64, 8), (128, 8), (128, 16)])
def test_q_high_norm_is_least_squares_residual(d, low_band):
    rng = np.random.default_rng(d + low_band)
    q = rng.standard_normal((5, d)).astype(np.float32)
    bs = d // low_band
    basis = np.kron(np.eye(low_band), np.ones((bs, 1)))  # block indicator vectors (d, low_band)
    for i in range(5):
        coef, *_ = np.linalg.lstsq(basis, q[i].astype(np.float64), rcond=None)
        resid = np.linalg.norm(q[i] - basis @ coef)
        np.testing.assert_allclose(O.q_high_norm_exact(q[i], low_band), resid, rtol=1e-5, atol=1e-5)
    # special cases: block-constant q has no high part; zero block sums keep all of it
    flat = np.repeat(rng.standard_normal(low_band), bs).astype(np.float32)
    assert O.q_high_norm_exact(flat, low_band) <= 1e-5 * np.linalg.norm(flat)
    zero_mean = q[0].reshape(low_band, bs) - q[0].reshape(low_band, bs).mean(axis=1, keepdims=True)
    np.testing.assert_allclose(O.q_high_norm_exact(zero_mean.reshape(-1), low_band),
                               np.linalg.norm(zero_mean), rtol=1e-5)


def test_decode_gate_rules():
    rng = np.random.default_rng(5)
    G, hkv, d, max_tiles, num_tiles = 4, 3, 64, 20, 17
    q = rng.standard_normal((hkv * G, d)).astype(np.float32)
    nc = rng.uniform(0.0, 100.0, size=(hkv, max_tiles)).astype(np.float32)
    tau = 0.01
    mask, qn = O.decode_gate(q, nc, tau, num_tiles, G)
    # the group's largest query norm, then one compare per tile
    for h in range(hkv):
        want = max(float(np.linalg.norm(q[h * G + g].astype(np.float64))) for g in range(G))
        np.testing.assert_allclose(qn[h], want, rtol=1e-6)
        for t in range(max_tiles):
            if t >= num_tiles:
                assert not mask[h, t]
            elif abs(qn[h] * nc[h, t] - tau * 64 * d) > 1e-3 * tau * 64 * d:
                assert mask[h, t] == (float(qn[h]) * float(nc[h, t]) <= tau * 64 * d)
    # thresholds at the extremes; zero queries evict every tile
    assert not O.decode_gate(q, nc, -1.0, num_tiles, G)[0].any()
    assert O.decode_gate(q, nc, 1e9, num_tiles, G)[0][:, :num_tiles].all()
    assert O.decode_gate(np.zeros_like(q), nc, 0.0, num_tiles, G)[0][:, :num_tiles].all()
    # tight: the Walsh-subspace norm, never above the spatial one
    _, qt = O.decode_gate(q, nc, tau, num_tiles, G, tight=True)
    assert (qt <= qn * (1 + 1e-6)).all()
    np.testing.assert_allclose(qt[1], max(O.q_high_norm_exact(q[G + g]) for g in range(G)), rtol=1e-6)


def test_apply_decode_mask_rules():
    rng = np.random.default_rng(6)
    G, hkv, s_len = 2, 3, 200  # 3 full tiles and a 8-token tail
    logits = rng.standard_normal((hkv * G, 1, s_len)).astype(np.float32)
    mask = np.zeros((hkv, 5), dtype=bool)
    mask[0, 1] = mask[2, 0] = mask[2, 3] = True
    out = O.apply_decode_mask(logits, mask, G)
    for h in range(hkv * G):
        for s in range(s_len):
            t = s // 64
            evicted = t < 3 and mask[h // G, t]
            assert (out[h, 0, s] == -np.inf) == evicted
            if not evicted:
                assert out[h, 0, s] == logits[h, 0, s]


@pytest.mark.parametrize("block_size", [64, 512])
def test_block_sparse_and_indirect_oracle(block_size):
    rng = np.random.default_rng(block_size)
    n_blocks, d = 6, 64
    q = rng.standard_normal((1, d)).astype(np.float32)
    k = rng.standard_normal((n_blocks * block_size, d)).astype(np.float32)
    v = rng.standard_normal((n_blocks * block_size, d)).astype(np.float32)
    mask = np.array([True, False, True, True, False, True])
    got = O.block_sparse_attention(q, k, v, mask, block_size)
    keep = np.repeat(mask, block_size)
    lg = (q.astype(np.float64) @ k[keep].T.astype(np.float64)) / np.sqrt(d)
    p = np.exp(lg - lg.max())
    want = (p / p.sum()) @ v[keep].astype(np.float64)
    np.testing.assert_allclose(got, want, atol=2e-6)
    np.testing.assert_allclose(O.block_sparse_attention(q, k, v, np.ones(n_blocks, bool), block_size),
                               O.dense_decode(q, k[None], v[None]), atol=2e-6)
    assert not O.block_sparse_attention(q, k, v, np.zeros(n_blocks, bool), block_size).any()
    idx = np.array([5, 0, 2, 3, 4], dtype=np.int32)
    np.testing.assert_allclose(O.indirect_attention(q, k, v, idx, 4, block_size), got, atol=2e-6)
    assert not O.indirect_attention(q, k, v, idx, 0, block_size).any()
