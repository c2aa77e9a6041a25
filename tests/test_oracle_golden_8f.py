"""CPU: the oracle's restatements of the paths around the decode reproduce
the vectors the reference's own CPU code wrote (tests/golden/make_golden_8f.py):
the decode gate's thresholds and q-norm forms, the norm cache, the
mask-given attention, the compact pipeline's auto tau, gates, statistics
and regimes, the eviction-regime classifier and the model hook's prefill
and decode branches with both governors.

Bars: masks, counts, regimes and retained sets exact; norms within 4
float32 ulps (a different summation order); outputs within the north-star
bar of the output dtype (tests/bars.py)."""

import numpy as np
import pytest

from oracle import orthocache_oracle as O
from tests import golden_io
from tests.bars import assert_out


@pytest.mark.parametrize("name,tight", [("gate_spatial", False), ("gate_high", True)])
def test_decode_gate_golden(name, tight):
    raw, dec, dt, meta, params, ref_fn = golden_io.load(name)
    mask, qn = O.decode_gate(dec["q"], dec["norm_cache"], params["tau"], params["num_tiles"], params["G"],
                             tight=tight, low_band=params["low_band"])
    assert np.array_equal(mask, dec["mask"].astype(bool))
    assert 0 < mask.sum() < mask.shape[0] * params["num_tiles"]
    np.testing.assert_allclose(qn, dec["q_norms"], rtol=4 * 2.0 ** -23)


def test_norm_cache_golden():
    raw, dec, dt, meta, params, _ = golden_io.load("norm_cache")
    lo, hi = params["band"]
    kn = O.band_norms(dec["keys"], lo, hi)
    T = kn.shape[1]
    np.testing.assert_allclose(kn, dec["bulk"][:, :T], rtol=4 * 2.0 ** -23)
    assert not dec["bulk"][:, T:].any()
    assert dec["valid_tiles"].tolist() == [T] * kn.shape[0]
    h, t = params["update"]
    np.testing.assert_allclose(O.band_norm(dec["tile"], lo, hi), dec["after"][h, t], rtol=4 * 2.0 ** -23)
    assert dec["valid_after"][h] == t + 1


@pytest.mark.parametrize("name", ["sparse_f32", "sparse_bf16"])
def test_block_sparse_and_indirect_golden(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    bs = params["block_size"]
    q, k, v = dec["q"], dec["keys"], dec["values"]
    got = O.block_sparse_attention(q, k, v, dec["block_mask"].astype(bool), bs)
    assert_out(got, dec["out_block_sparse"], "f32", f"oracle block sparse {name}")
    got = O.indirect_attention(q, k, v, dec["active_indices"], params["num_active"], bs)
    assert_out(got, dec["out_indirect"], "f32", f"oracle indirect {name}")


@pytest.mark.parametrize("name", ["compact_f32", "compact"])
def test_compact_forward_golden(name):
    """float32: auto tau, zeta statistics and counts to float32 rounding;
    bfloat16: the reference computes its spectra and statistics in the
    input dtype, so only the decisions are exact and the statistics agree
    to bfloat16 rounding (2^-8 relative, accumulated)."""
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    q, k, v = dec["q"], dec["keys"], dec["values"]
    stat_rtol = 1e-5 if name == "compact_f32" else 2e-2
    for tau_name in ("auto", "given"):
        m = meta[tau_name]
        tau = None if tau_name == "auto" else params["tau_given"]
        out, info = O.compact_forward(q, k, v, zeta_max=params["zeta_max"], tau=tau)
        assert info["retained"] == m["blocks_retained"]
        assert info["perfect"] == m["perfect_eviction_blocks"]
        assert info["statistical"] == m["statistical_eviction_blocks"]
        assert info["tau"] == pytest.approx(m["tau"], rel=stat_rtol)
        for key in ("zeta_mean", "zeta_std", "zeta_min", "zeta_max_observed"):
            assert info[key] == pytest.approx(m[key], rel=stat_rtol), key
        out_dt = dt["out_" + tau_name]
        assert_out(O.round_to(out.astype(np.float32), out_dt) if out_dt != "f32" else out,
                   dec["out_" + tau_name], out_dt, f"oracle compact {name} {tau_name}", ref_rounded=True,
                   out_dtype=out_dt)


def test_regimes_golden():
    raw, dec, dt, meta, params, _ = golden_io.load("regimes")
    reg, beta, gap, full, counts = O.block_regimes(dec["q"], dec["energy"], params["head_dim"], dec["z_max"],
                                                   dec["mask"].astype(bool))
    assert np.array_equal(reg, dec["regime"]) and list(counts) == meta["counts"]
    np.testing.assert_allclose(full, dec["beta_full"], rtol=4 * 2.0 ** -23)
    np.testing.assert_allclose(beta, dec["beta"], rtol=4 * 2.0 ** -23)
    np.testing.assert_allclose(gap, dec["gap"], rtol=4 * 2.0 ** -23, atol=1e-4)
    reg, _, gap, _, counts = O.block_regimes(dec["q"], dec["energy"], params["head_dim"], params["z_max_b"],
                                             dec["mask"].astype(bool).any(axis=1), meta["threshold_b"])
    assert np.array_equal(reg, dec["regime_b"]) and list(counts) == meta["counts_b"]
    np.testing.assert_allclose(gap, dec["gap_b"], rtol=4 * 2.0 ** -23, atol=1e-4)


def hook_inputs(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    src = params.get("inputs_from", name)
    inp = golden_io.load(src)[1]
    return inp, dec, meta, params


@pytest.mark.parametrize("name", ["hook_residual", "hook_entropy"])
def test_hook_golden(name):
    """The hook's prefill then one decode step, driven through the oracle
    with the governor arithmetic of the reference: every batch element
    reports its eviction rate to the governor, and the call's tau is taken
    once before the batch loop (perplexity_eval.py:407-411, :508-512,
    :580-584, :659-662)."""
    inp, dec, meta, params = hook_inputs(name)
    G, tau, alpha = params["G"], params["tau"], params["alpha"]
    entropy_gov = name == "hook_entropy"
    rates, entropy = [], None

    def tau_eff():
        if entropy_gov:
            return O.entropy_tau(tau, alpha, rates, params["beta"], params["h_median"], entropy)
        return O.residual_tau(tau, alpha, rates)

    qp, kp, vp = inp["q_prefill"], inp["k_prefill"], inp["v_prefill"]
    B, Hkv, S = kp.shape[0], kp.shape[1], kp.shape[2]
    T = S // 64
    pre = O.hook_prefill(qp, kp, vp, G, tau_eff())
    assert_out(pre["out"], dec["out_prefill"], "f32", f"oracle {name} prefill")
    for b in range(B):
        rates.append(pre["evicted"][b] / (Hkv * T))
        if entropy_gov:
            entropy = float(pre["entropy"][b])
    # the reference averages the entropy in float32 (a tensor mean), the
    # oracle in float64: the entropy governor's tau agrees to float32 rounding
    rel = 1e-6 if entropy_gov else 1e-12
    assert meta["tau_after_prefill"] == pytest.approx(tau_eff(), rel=rel)
    nc = pre["k_norms"][B - 1]  # the cache holds the last batch element's norms
    np.testing.assert_allclose(nc, dec["norm_cache"][:, :T], rtol=4 * 2.0 ** -23)
    assert dec["valid_tiles"].tolist() == [T] * Hkv
    dd = O.hook_decode(inp["q_decode"], inp["k_decode"], inp["v_decode"], nc, G, tau_eff())
    assert_out(dd["out"], dec["out_decode"], "f32", f"oracle {name} decode")
    for b in range(B):
        rates.append(dd["skipped"][b] / (Hkv * T))
    assert meta["layer_history"] == pytest.approx(rates, rel=1e-12)
    assert meta["tau_after_decode"] == pytest.approx(tau_eff(), rel=rel, abs=1e-15)
    assert meta["evicted_tiles"] == int(pre["evicted"].sum())
    assert meta["total_tiles"] == B * Hkv * T
    assert meta["decode_tiles_skipped"] == int(dd["skipped"].sum())
    assert meta["decode_steps"] == B and meta["decode_tiles_total"] == B * Hkv * T
    np.testing.assert_allclose(meta["hallucination_scores"], np.concatenate([pre["h_score"], dd["h_score"]]),
                               rtol=1e-6)
    np.testing.assert_allclose(meta["q_search_intensity"], np.concatenate([pre["max_q"], dd["max_q"]]), rtol=1e-6)
    np.testing.assert_allclose(meta["k_info_density"], np.concatenate([pre["max_k"], dd["max_k"]]), rtol=1e-6)
    if entropy_gov:
        assert meta["entropy"] == pytest.approx(float(pre["entropy"][B - 1]), rel=1e-5)
