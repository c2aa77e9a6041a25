"""Pins of the oracle's model-hook functions (CPU only): causal attention
against explicit per-query loops, eviction against attention over the kept
keys, the entropy of uniform attention, the median rank rules against
torch.median and explicit lists, the [48, 64) band against its closed form,
the gate's threshold extremes, and the governors' closed forms."""

import math

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O


def _qkv(B, Hq, Hkv, Sq, Skv, d, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, d)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Skv, d)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Skv, d)).astype(np.float32)
    return q, k, v


def _loop_attention(qv, keys, values, scale):
    """softmax(q.k * scale) @ v by explicit sums (math.exp)."""
    lg = [float(np.dot(qv.astype(np.float64), kk.astype(np.float64))) * scale for kk in keys]
    m = max(lg)
    w = [math.exp(x - m) for x in lg]
    z = sum(w)
    return sum(wi * vv.astype(np.float64) for wi, vv in zip(w, values)) / z


@pytest.mark.parametrize("Sq,Skv", [(5, 5), (3, 70), (70, 70)])
def test_causal_attention_matches_per_query_loops(Sq, Skv):
    G, d = 2, 8
    q, k, v = _qkv(1, 4, 2, Sq, Skv, d, Sq + Skv)
    out, _ = O.hook_causal_attention(q, k, v, G)
    for h in range(4):
        for s in range(Sq):
            n = s + Skv - Sq + 1
            want = _loop_attention(q[0, h, s], k[0, h // G, :n], v[0, h // G, :n], 1 / math.sqrt(d))
            np.testing.assert_allclose(out[0, h, s], want, rtol=1e-10, atol=1e-12)


def test_eviction_is_attention_over_kept_keys():
    G, d, S = 2, 16, 200  # 3 complete tiles and a partial one
    q, k, v = _qkv(1, 2, 1, 1, S, d, 3)
    evict = np.array([[[True, False, True]]])
    out, _ = O.hook_causal_attention(q, k, v, G, evict)
    keep = np.r_[64:128, 192:200]
    for h in range(2):
        want = _loop_attention(q[0, h, 0], k[0, 0, keep], v[0, 0, keep], 1 / math.sqrt(d))
        np.testing.assert_allclose(out[0, h, 0], want, rtol=1e-10, atol=1e-12)
    # every complete tile evicted: only the partial tile's 8 keys are left
    out2, _ = O.hook_causal_attention(q, k, v, G, np.ones((1, 1, 3), bool))
    want = _loop_attention(q[0, 0, 0], k[0, 0, 192:], v[0, 0, 192:], 1 / math.sqrt(d))
    np.testing.assert_allclose(out2[0, 0, 0], want, rtol=1e-10)
    # a query that sees no key (more queries than keys) gets zeros
    q3, k3, v3 = _qkv(1, 1, 1, 6, 4, d, 4)
    out3, ent3 = O.hook_causal_attention(q3, k3, v3, 1)
    assert not out3[0, 0, :2].any() and out3[0, 0, 2:].any()
    np.testing.assert_allclose(ent3[0, 0, 0], 4 * 1e-10 * math.log(1e10), rtol=1e-12)


def test_entropy_of_uniform_attention():
    d, S = 8, 100
    _, k, v = _qkv(1, 1, 1, 1, S, d, 5)
    q = np.zeros((1, 1, 3, d), np.float32)  # logits all 0: uniform over the visible keys
    _, ent = O.hook_causal_attention(q, k, v, 1)
    for s in range(3):
        n = s + S - 3 + 1
        want = math.log(n) + (S - n) * 1e-10 * math.log(1e10)
        np.testing.assert_allclose(ent[0, 0, s], want, rtol=1e-12)


def test_median_rules():
    rng = np.random.default_rng(7)
    for n in (1, 2, 5, 8, 33):
        x = rng.random((4, n)).astype(np.float32)
        assert np.array_equal(O.torch_lower_median(x), torch.from_numpy(x).median(dim=1).values.numpy())
    assert O.torch_lower_median(np.array([4.0, 1.0, 3.0, 2.0])) == 2.0
    # the decode branch: sorted(group)[G // 2], the upper median for even G
    qh = np.array([[4.0, 1.0, 3.0, 2.0]], np.float32)
    assert np.sort(qh, axis=1)[:, 2] == 3.0


def test_hook_tile_norms_closed_form_and_no_clamp():
    rng = np.random.default_rng(8)
    keys = rng.standard_normal((1, 2, 130, 16)).astype(np.float32)
    kn = O.hook_tile_norms(keys)
    assert kn.shape == (1, 2, 2)
    for h in range(2):
        for t in range(2):
            kt = keys[0, h, 64 * t:64 * t + 64].astype(np.float64)
            g = kt[0:16] - kt[16:32] - kt[32:48] + kt[48:64]
            # rows 48..63 of the unnormalised H64: 16 sum ||g||^2 (64x the W64 band)
            np.testing.assert_allclose(kn[0, h, t], np.sqrt(16.0 * np.sum(g ** 2)), rtol=2e-6)
            # exactly 8x the normalised band norm (a power-of-two scale)
            assert kn[0, h, t] == np.float32(8.0) * O.band_norm(keys[0, h, 64 * t:64 * t + 64], 48, 64)
    # a float32 sum of squares is 0 or >= 2^-149, so its root is 0 or above
    # 3e-23: the 1e-38 clamp of SpectralNormCache never changes a float32 norm
    tiny = np.zeros((1, 1, 64, 4), np.float32)
    tiny[0, 0, 0, 0] = 1e-18
    assert O.hook_tile_norms(tiny)[0, 0, 0] == 8 * O.band_norm(tiny[0, 0], 48, 64) > 1e-38


def test_hook_prefill_gate_extremes_and_stats():
    q, k, v = _qkv(2, 4, 2, 70, 200, 16, 9)
    G = 2
    none = O.hook_prefill(q, k, v, G, tau=-1.0)
    assert not none["evict"].any()
    plain, ent = O.hook_causal_attention(q, k, v, G)
    np.testing.assert_allclose(none["out"], plain, rtol=1e-12)
    np.testing.assert_allclose(none["entropy"], ent.reshape(2, -1).mean(axis=1), rtol=1e-12)
    allv = O.hook_prefill(q, k, v, G, tau=1e30)
    assert allv["evict"].all() and list(allv["evicted"]) == [2 * 3, 2 * 3]
    # the gate itself: qn = max over the group of the lower medians over positions
    qnorm = np.linalg.norm(q.astype(np.float64), axis=-1)
    med = np.sort(qnorm, axis=-1)[..., (70 - 1) // 2]
    np.testing.assert_allclose(none["qn"], med.reshape(2, 2, G).max(axis=2), rtol=1e-6)
    mid = float(np.median(none["qn"][:, :, None] * none["k_norms"])) / (64 * 16)
    some = O.hook_prefill(q, k, v, G, tau=mid)
    prods = none["qn"][:, :, None].astype(np.float64) * none["k_norms"] / (64 * 16)
    assert np.array_equal(some["evict"], prods <= mid)
    np.testing.assert_allclose(some["h_score"], some["max_q"] / (some["max_k"] + 1e-10))


def test_hook_decode_gate():
    q, k, v = _qkv(2, 8, 2, 1, 200, 16, 10)
    G = 4
    nc = np.random.default_rng(1).uniform(0, 40, size=(2, 5)).astype(np.float32)
    res = O.hook_decode(q, k, v, nc, G, tau=0.5)
    qh = O.q_high_norm_exact(q[:, :, 0])
    for b in range(2):
        for h in range(2):
            qn = sorted(qh[b, h * G:(h + 1) * G].tolist())[G // 2]
            assert res["qn"][b, h] == np.float32(qn)
            for t in range(3):  # 200 tokens: 3 complete tiles
                assert res["evict"][b, h, t] == (qn * float(nc[h, t]) / (64 * 16) <= 0.5)
    allv = O.hook_decode(q, k, v, nc, G, tau=1e30)
    out, _ = O.hook_causal_attention(q, k, v, G, np.ones((2, 2, 3), bool))
    np.testing.assert_allclose(allv["out"], out)
    assert list(allv["skipped"]) == [6, 6]


def test_governor_closed_forms():
    assert O.residual_tau(2.0, 0.5, [0.2, 0.3]) == 2.0 * 0.75
    assert O.residual_tau(2.0, 1.0, [0.7, 0.6]) == 0.0
    assert O.entropy_tau(1.0, 0.5, [], 1.0, 1.56, 1.56) == 1.0
    assert O.entropy_tau(1.0, 0.5, [], 1.0, 1.56, None) == 1.0
    np.testing.assert_allclose(O.entropy_tau(1.0, 0.0, [], 2.0, 1.0, 1.5), 2.0 / (1.0 + math.exp(-1.0)))
