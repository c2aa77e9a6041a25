"""GPU: the HIP path of the paths around the decode against the vectors the
reference's own CPU code wrote (tests/golden/make_golden_8f.py): the O(1)
decode gate (spatial and Walsh-subspace q norms), the norm cache (bulk and
per tile, normalised and unnormalised Walsh matrices), block-sparse and
indirect attention, orthocache_forward(mode='compact') (float32: decisions,
auto tau and statistics; bfloat16: decisions, statistics to the
reference's bfloat16 rounding), the eviction-regime classifier and the
model hook's prefill and decode steps with both governors.

Bars: masks, counts, regimes and retained sets exact; norms within 4
float32 ulps; outputs within the north-star bar (tests/bars.py)."""

import numpy as np
import pytest
import torch

from tests import golden_io
from tests.bars import assert_out

pytestmark = pytest.mark.gpu
DEV = "cuda"
ULP4 = 4 * 2.0 ** -23


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield


def dev(raw, dt):
    """stored bits -> device tensor of the stored dtype"""
    if dt == "f32":
        return torch.from_numpy(raw.astype(np.float32)).to(DEV)
    if dt in ("f16", "bf16"):
        t = torch.from_numpy(raw.astype(np.uint16).view(np.int16))
        return t.view(torch.float16 if dt == "f16" else torch.bfloat16).to(DEV)
    if dt == "i32":
        return torch.from_numpy(raw.astype(np.int32)).to(DEV)
    if dt == "bool":
        return torch.from_numpy(raw.astype(bool)).to(DEV)
    raise ValueError(dt)


def load(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    return {k: dev(raw[k], dt[k]) for k in raw}, dec, dt, meta, params


def np64(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("name,q_norm", [("gate_spatial", "spatial"), ("gate_high", "high")])
def test_decode_gate(name, q_norm):
    from orthocache_gpu.triton_kernels.decode_gate import decode_gate
    t, dec, dt, meta, params = load(name)
    mask, qn = decode_gate(t["q"], t["norm_cache"], params["tau"], params["num_tiles"], params["G"],
                           q_norm=q_norm, low_band=params["low_band"])
    assert np.array_equal(mask.cpu().numpy(), dec["mask"].astype(bool))
    np.testing.assert_allclose(np64(qn), dec["q_norms"], rtol=ULP4)


def test_norm_cache():
    from orthocache_gpu import generate_walsh_matrix
    from orthocache_gpu.norm_cache import SpectralNormCache
    t, dec, dt, meta, params = load("norm_cache")
    lo, hi = params["band"]
    hkv = t["keys"].shape[0]
    w = generate_walsh_matrix(64).to(DEV)
    cache = SpectralNormCache(hkv, params["max_tiles"], torch.device(DEV))
    cache.populate_from_keys(t["keys"], w, 64, lo, hi)
    np.testing.assert_allclose(np64(cache.cache), dec["bulk"], rtol=ULP4)
    assert cache.valid_tiles.cpu().tolist() == dec["valid_tiles"].tolist()
    bulk = cache.cache.clone()
    h, tile = params["update"]
    cache.update_prefill(h, tile, t["tile"], w, lo, hi)
    np.testing.assert_allclose(np64(cache.cache), dec["after"], rtol=ULP4)
    assert cache.valid_tiles.cpu().tolist() == dec["valid_after"].tolist()
    # the reference's evaluation code uses the unnormalised H64 (8 x W64):
    # the same norms scaled by exactly 8
    c8 = SpectralNormCache(hkv, params["max_tiles"], torch.device(DEV))
    c8.populate_from_keys(t["keys"], w * 8.0, 64, lo, hi)
    assert torch.equal(c8.cache, bulk * 8.0)
    with pytest.raises(NotImplementedError):
        c8.populate_from_keys(t["keys"], torch.ones(64, 64, device=DEV), 64, lo, hi)


@pytest.mark.parametrize("name", ["sparse_f32", "sparse_bf16"])
def test_block_sparse_and_indirect(name):
    from orthocache_gpu.triton_kernels import triton_block_sparse_attention, triton_indirect_attention
    t, dec, dt, meta, params = load(name)
    bs = params["block_size"]
    bar = dt["q"]
    out = triton_block_sparse_attention(t["q"], t["keys"], t["values"], t["block_mask"], bs)
    assert out.dtype == t["q"].dtype
    assert_out(out, dec["out_block_sparse"], bar, f"golden block sparse {name}")
    out = triton_indirect_attention(t["q"], t["keys"], t["values"], t["active_indices"], params["num_active"], bs)
    assert_out(out, dec["out_indirect"], bar, f"golden indirect {name}")


@pytest.mark.parametrize("name", ["compact_f32", "compact"])
def test_compact_forward(name):
    """Decisions exact; auto tau and zeta statistics to float32 rounding
    (float32 inputs) or to the reference's bfloat16 arithmetic (bfloat16
    inputs: it forms its spectra and statistics in the input dtype, this
    build in float32)."""
    from orthocache_gpu import orthocache_forward
    t, dec, dt, meta, params = load(name)
    rtol = 1e-5 if name == "compact_f32" else 2e-2
    for tau_name in ("auto", "given"):
        m = meta[tau_name]
        tau = None if tau_name == "auto" else params["tau_given"]
        out, got = orthocache_forward(t["q"], t["keys"], t["values"], block_size=params["block_size"],
                                      zeta_max=params["zeta_max"], tau=tau, mode="compact")
        assert got["actual_mode"] == "compact"
        for key in ("blocks_retained", "blocks_evicted", "compact_num_active", "perfect_eviction_blocks",
                    "statistical_eviction_blocks", "num_blocks", "tau_auto"):
            assert got[key] == m[key], key
        assert got["eviction_rate"] == pytest.approx(m["eviction_rate"])
        for key in ("tau", "zeta_mean", "zeta_std", "zeta_min", "zeta_max_observed"):
            assert got[key] == pytest.approx(m[key], rel=rtol), key
        # both return bfloat16 whatever the input dtype (adaptive_attention.py)
        assert dt["out_" + tau_name] == "bf16" and out.dtype == torch.bfloat16
        assert_out(out, dec["out_" + tau_name], "bf16", f"golden compact {name} {tau_name}", ref_rounded=True)


def test_regimes():
    from orthocache_gpu.perfect_eviction import classify_eviction, compute_block_beta
    t, dec, dt, meta, params = load("regimes")
    d = params["head_dim"]
    beta = compute_block_beta(t["q"], t["energy"], d)
    np.testing.assert_allclose(np64(beta), dec["beta_full"], rtol=ULP4)
    m = classify_eviction(t["q"], t["energy"], t["z_max"], t["mask"], d)
    assert np.array_equal(m.regime.cpu().numpy(), dec["regime"])
    assert [m.num_perfect, m.num_statistical, m.num_retained] == meta["counts"]
    assert m.underflow_threshold == meta["threshold"]
    np.testing.assert_allclose(np64(m.beta), dec["beta"], rtol=ULP4)
    np.testing.assert_allclose(np64(m.logit_gap), dec["gap"], rtol=ULP4, atol=1e-4)
    m = classify_eviction(t["q"], t["energy"], torch.tensor(params["z_max_b"]), t["mask"].any(dim=1), d,
                          accumulator_dtype="bfloat16")
    assert np.array_equal(m.regime.cpu().numpy(), dec["regime_b"])
    assert [m.num_perfect, m.num_statistical, m.num_retained] == meta["counts_b"]
    assert m.underflow_threshold == meta["threshold_b"]


@pytest.mark.parametrize("name", ["hook_residual", "hook_entropy"])
def test_model_hook(name):
    """Prefill (4 tiles per row, half evicted) then one decode step over a
    partial fifth tile, batch 2, G = 2: outputs, norm cache, statistics and
    the governor's per-element eviction rates and tau against the
    reference's own run."""
    from orthocache_gpu.model_hook import EntropyGovernor, OrthoCache_GQA_Attention, ResidualGovernor
    from orthocache_gpu.norm_cache import SpectralNormCache
    _, dec, dt, meta, params = load(name)
    src = params.get("inputs_from", name)
    inp, _, _, _, _ = load(src)
    G, tau = params["G"], params["tau"]
    if name == "hook_entropy":
        gov = EntropyGovernor(alpha=params["alpha"], beta=params["beta"], h_median=params["h_median"])
    else:
        gov = ResidualGovernor(alpha=params["alpha"])
    hook = OrthoCache_GQA_Attention(tau=tau, governor=gov)
    Hkv = inp["k_prefill"].shape[1]
    hook.norm_cache = SpectralNormCache(Hkv, dec["norm_cache"].shape[1], torch.device(DEV))
    out_p = hook.orthocache_attention(inp["q_prefill"], inp["k_prefill"], inp["v_prefill"], G)
    assert_out(out_p, dec["out_prefill"], "f32", f"golden {name} prefill")
    rel = 1e-6 if name == "hook_entropy" else 1e-12  # entropy: a float32 mean in both
    assert gov.get_tau_effective(tau) == pytest.approx(meta["tau_after_prefill"], rel=rel)
    np.testing.assert_allclose(np64(hook.norm_cache.cache), dec["norm_cache"], rtol=ULP4)
    assert hook.norm_cache.valid_tiles.cpu().tolist() == dec["valid_tiles"].tolist()
    out_d = hook.orthocache_attention(inp["q_decode"], inp["k_decode"], inp["v_decode"], G)
    assert_out(out_d, dec["out_decode"], "f32", f"golden {name} decode")
    st = hook.stats
    for key in ("total_tiles", "evicted_tiles", "layers_processed", "decode_steps", "decode_tiles_skipped",
                "decode_tiles_total"):
        assert st[key] == meta[key], key
    for key in ("hallucination_scores", "q_search_intensity", "k_info_density"):
        np.testing.assert_allclose(st[key], meta[key], rtol=2e-6, err_msg=key)
    assert gov.layer_history == pytest.approx(meta["layer_history"], rel=1e-12)
    assert gov.get_tau_effective(tau) == pytest.approx(meta["tau_after_decode"], rel=rel, abs=1e-15)
    if name == "hook_entropy":
        assert st["entropy"] == pytest.approx(meta["entropy"], rel=1e-5)
