"""GPU parity of the model-side hook (OrthoCache_GQA_Attention and its
kernels) against the oracle: oc_prefill_attention (causal GQA attention
with evicted tiles and the attention entropy), oc_row_norms,
oc_kth_smallest, oc_group_gate, the hook's prefill and decode branches
call for call (outputs, statistics, norm cache, governor), and a
transformers Llama model patched with the hook.

Bars: float32 outputs within 1e-5 (+1e-5 relative); float16 / bfloat16
outputs within 2e-3 plus half an output ulp of the float64 oracle; masks and
selections bit-exact (thresholds placed away from every decision); entropy
within 1e-4.
"""

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O
from tests.bars import assert_out

pytestmark = pytest.mark.gpu
DEV = "cuda"
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield


def np64(t):
    return t.detach().double().cpu().numpy()


def _qkv(B, Hq, Hkv, Sq, Skv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Sq, Hq, d), generator=g).to(TD[dtype]).to(DEV)
    k = torch.randn((B, Hkv, Skv + 5, d), generator=g).to(TD[dtype]).to(DEV)
    v = torch.randn((B, Hkv, Skv, d), generator=g).to(TD[dtype]).to(DEV)
    # q as the (B, S, H, d) -> (B, H, S, d) view a decoder layer passes; k a
    # slice of a longer cache (strides of Skv + 5 tokens)
    return q.transpose(1, 2), k[:, :, :Skv], v


CASES = [  # B, Hq, Hkv, Sq, Skv, d
    (2, 8, 2, 200, 200, 64),    # prefill with a partial last tile
    (1, 4, 4, 37, 300, 128),    # chunk of queries at the end of a longer context
    (1, 4, 1, 100, 64, 64),     # more queries than keys: the first 36 see none
    (2, 8, 2, 1, 333, 128),     # one query
    (1, 16, 2, 130, 130, 128),  # G = 8
]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("masked", [False, True])
def test_prefill_attention_vs_oracle(dtype, case, masked):
    from orthocache_gpu import _launch as X
    B, Hq, Hkv, Sq, Skv, d = case
    G = Hq // Hkv
    q, k, v = _qkv(B, Hq, Hkv, Sq, Skv, d, dtype, seed=sum(case))
    evict = None
    tm = None
    if masked:
        evict = torch.rand((B, Hkv, Skv // 64), generator=torch.Generator().manual_seed(3)) < 0.5
        tm = evict.to(torch.uint8).to(DEV)
    print(f"prefill {dtype} {case} masked={masked}", flush=True)
    out, ent = X.prefill_attention(q, k, v, tile_mask=tm, want_entropy=True)
    torch.cuda.synchronize()
    ref, ref_ent = O.hook_causal_attention(np64(q), np64(k), np64(v), G,
                                           None if evict is None else evict.numpy())
    assert out.dtype == q.dtype and out.shape == (B, Hq, Sq, d)
    assert_out(out, ref, dtype, f"prefill {dtype} {case} masked={masked}")
    np.testing.assert_allclose(np64(ent), ref_ent, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("masked", [False, True])
def test_prefill_split_windows_vs_oracle(dtype, d, masked):
    """A call whose workgroups fit the device in one round, with no tiles
    evicted, runs its longest causal windows as two workgroups each (the
    second to finish merges the two halves' states); output and entropy match
    the oracle as the unsplit call's do, and the library asked for a
    workspace (so it did split).  A masked call does not split."""
    import ctypes
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    B, Hq, Hkv, S = 1, 8, 2, 1000  # 8 query blocks, windows of 2..16 tiles
    G = Hq // Hkv
    q, k, v = _qkv(B, Hq, Hkv, S, S, d, dtype, seed=d + (7 if masked else 0))
    evict, tm = None, None
    if masked:
        evict = torch.rand((B, Hkv, S // 64), generator=torch.Generator().manual_seed(5)) < 0.4
        tm = evict.to(torch.uint8).to(DEV)
    p = N.OcPrefillParams()
    p.dtype, p.batch, p.num_q_heads, p.num_kv_heads = X.dtype_code(q.dtype, "q"), B, Hq, Hkv
    p.q_len, p.kv_len, p.head_dim = S, S, d
    if masked:
        p.tile_mask, p.tile_mask_cols = tm.data_ptr(), S // 64
    # a mask turns the split off (its merge does not pay with tiles evicted)
    assert (N.lib().oc_prefill_workspace_size(ctypes.byref(p)) > 0) == (not masked)
    print(f"prefill split {dtype} d={d} masked={masked}", flush=True)
    out, ent = X.prefill_attention(q, k, v, tile_mask=tm, want_entropy=True)
    out1, ent1 = X.prefill_attention(q, k, v, tile_mask=tm, want_entropy=True, split=False)
    torch.cuda.synchronize()
    ref, ref_ent = O.hook_causal_attention(np64(q), np64(k), np64(v), G,
                                           None if evict is None else evict.numpy())
    for o, e, what in ((out, ent, "split"), (out1, ent1, "one workgroup per block")):
        assert_out(o, ref, dtype, f"prefill {what} {dtype} d={d} masked={masked}")
        np.testing.assert_allclose(np64(e), ref_ent, atol=1e-4, rtol=1e-5)
    # a second call reuses the workspace (its tickets were left at zero)
    out2, ent2 = X.prefill_attention(q, k, v, tile_mask=tm, want_entropy=True)
    assert torch.equal(out2, out) and torch.equal(ent2, ent)


SPLIT_CASES = [  # B, Hq, Hkv, Sq, Skv, d: calls that split their longest windows
    (2, 4, 4, 300, 700, 64),    # chunk of queries at the end of a longer context, G = 1
    (1, 16, 2, 513, 513, 128),  # G = 8, a partial last query block and tile
    (1, 8, 1, 37, 2000, 64),    # one query block, a 32-tile window
    (2, 8, 2, 640, 640, 128),   # five query blocks per head
]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "x".join(map(str, c)))
def test_prefill_split_shapes_vs_oracle(dtype, case):
    import ctypes
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    B, Hq, Hkv, Sq, Skv, d = case
    q, k, v = _qkv(B, Hq, Hkv, Sq, Skv, d, dtype, seed=sum(case) + 1)
    p = N.OcPrefillParams()
    p.dtype, p.batch, p.num_q_heads, p.num_kv_heads = X.dtype_code(q.dtype, "q"), B, Hq, Hkv
    p.q_len, p.kv_len, p.head_dim = Sq, Skv, d
    assert N.lib().oc_prefill_workspace_size(ctypes.byref(p)) > 0
    print(f"prefill split {dtype} {case}", flush=True)
    out, ent = X.prefill_attention(q, k, v, want_entropy=True)
    torch.cuda.synchronize()
    ref, ref_ent = O.hook_causal_attention(np64(q), np64(k), np64(v), Hq // Hkv, None)
    assert_out(out, ref, dtype, f"prefill split {dtype} {case}")
    np.testing.assert_allclose(np64(ent), ref_ent, atol=1e-4, rtol=1e-5)


def test_row_norms_and_selection():
    from orthocache_gpu import _launch as X
    g = torch.Generator().manual_seed(4)
    x = torch.randn((2, 70, 6, 64), generator=g).transpose(1, 2).to(DEV)  # (2, 6, 70, 64) strided
    got = X.row_norms(x)
    np.testing.assert_allclose(np64(got), np.linalg.norm(np64(x), axis=-1), rtol=2e-6)
    hi = X.row_norms(x, low_band=8)
    np.testing.assert_allclose(np64(hi), O.q_high_norm_exact(x.float().cpu().numpy(), 8), rtol=8 * 2.0 ** -23,
                               atol=1e-6)
    for n in (1, 2, 7, 1000, 4097):
        vals = torch.rand((5, n), generator=g) * 10
        vals[:, ::3] = vals[:, ::3].round()  # ties
        vals[1, :n // 2] = 0.0
        srt = np.sort(vals.numpy(), axis=1)
        for k in {0, (n - 1) // 2, n - 1}:
            sel = X.kth_smallest(vals.to(DEV), k)
            assert np.array_equal(sel.cpu().numpy(), srt[:, k]), (n, k)


@pytest.mark.parametrize("reduce", ["max", "median"])
def test_group_gate_vs_loops(reduce):
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rng = np.random.default_rng(5)
    B, Hkv, G, T, cols = 3, 4, 4, 37, 40
    qn = rng.uniform(0, 20, size=(B, Hkv * G)).astype(np.float32)
    kn = rng.uniform(0, 30, size=(B, Hkv, 48)).astype(np.float32)
    tau_norm = 150.0
    mode = N.OC_GROUP_MAX if reduce == "max" else N.OC_GROUP_MEDIAN
    for keep in (False, True):
        for shared in (False, True):
            kn_t = torch.from_numpy(kn[:1] if shared else kn).to(DEV)
            mask, gn, st = X.group_gate(torch.from_numpy(qn).to(DEV), kn_t, Hkv, G, T, cols, tau_norm, mode,
                                        keep_polarity=keep, want_stats=True)
            mask, gn, st = mask.cpu().numpy(), gn.cpu().numpy(), st.cpu().numpy()
            for b in range(B):
                for h in range(Hkv):
                    grp = qn[b, h * G:(h + 1) * G]
                    want = grp.max() if reduce == "max" else np.sort(grp)[G // 2]
                    assert gn[b, h] == want
                    knr = kn[0 if shared else b, h]
                    evs = [t < T and np.float32(want) * knr[t] <= np.float32(tau_norm) for t in range(cols)]
                    for t in range(cols):
                        assert mask[b, h, t] == (int(not evs[t]) if keep else int(evs[t]))
                    # the hook's per-call statistics before their reductions
                    assert st[b, h, 0] == sum(evs) and st[b, h, 1] == want and st[b, h, 2] == knr[:T].max()


def test_group_gate_stats_edge_cases():
    """The gate statistics with no complete tile (-inf K maximum) and with a
    NaN K norm (NaN, as torch's amax gives)."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    qn = torch.ones((1, 4), device=DEV)
    kn = torch.ones((1, 2, 8), device=DEV)
    _, _, st = X.group_gate(qn, kn, 2, 2, 0, 1, 1.0, N.OC_GROUP_MAX, keep_polarity=True, want_stats=True)
    st = st.cpu().numpy()
    assert (st[0, :, 0] == 0).all() and np.isneginf(st[0, :, 2]).all()
    kn[0, 1, 3] = float("nan")
    _, _, st = X.group_gate(qn, kn, 2, 2, 8, 8, 1.0, N.OC_GROUP_MAX, keep_polarity=True, want_stats=True)
    st = st.cpu().numpy()
    assert st[0, 0, 2] == 1.0 and np.isnan(st[0, 1, 2])


def _gap_tau(prods):
    """a threshold in the widest relative gap of the middle half of prods"""
    p = np.sort(prods.ravel())
    p = p[p > 0]
    lo, hi = len(p) // 4, 3 * len(p) // 4
    gaps = p[lo + 1:hi + 1] / p[lo:hi]
    i = lo + int(np.argmax(gaps))
    assert p[i + 1] / p[i] > 1 + 1e-4
    return float(np.sqrt(p[i] * p[i + 1]))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_hook_prefill_then_decode_vs_oracle(dtype):
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention, ResidualGovernor
    from orthocache_gpu.norm_cache import SpectralNormCache
    B, Hq, Hkv, d, S = 2, 8, 2, 64, 320
    G = Hq // Hkv
    q, k, v = _qkv(B, Hq, Hkv, S, S + 10, d, dtype, seed=11)
    kp, vp = k[:, :, :S], v[:, :, :S]
    probe = O.hook_prefill(np64(q), np64(kp), np64(vp), G, tau=-1.0)
    tau = _gap_tau(probe["qn"][:, :, None].astype(np.float64) * probe["k_norms"] / (64 * d))
    gov = ResidualGovernor(alpha=0.5)
    hook = OrthoCache_GQA_Attention(tau=tau, governor=gov)
    hook.norm_cache = SpectralNormCache(Hkv, 16, torch.device(DEV))
    print(f"hook prefill {dtype} tau={tau}", flush=True)
    out = hook.orthocache_attention(q, kp, vp, G)
    ref = O.hook_prefill(np64(q), np64(kp), np64(vp), G, tau)
    assert_out(out, ref["out"], dtype, f"hook prefill {dtype}")
    T = S // 64
    assert 0 < ref["evict"].sum() < B * Hkv * T
    assert hook.stats['total_tiles'] == B * Hkv * T
    assert hook.stats['evicted_tiles'] == int(ref["evicted"].sum())
    np.testing.assert_allclose(hook.stats['hallucination_scores'], ref["h_score"], rtol=1e-5)
    np.testing.assert_allclose(hook.stats['q_search_intensity'], ref["max_q"], rtol=1e-5)
    np.testing.assert_allclose(hook.stats['k_info_density'], ref["max_k"], rtol=1e-5)
    np.testing.assert_allclose(gov.layer_history, ref["evicted"] / (Hkv * T), rtol=1e-12)
    nc = hook.norm_cache
    np.testing.assert_allclose(np64(nc.cache[:, :T]), ref["k_norms"][B - 1], rtol=4 * 2.0 ** -23)
    assert nc.valid_tiles.cpu().tolist() == [T, T] and nc.is_populated
    # decode: one query per head over 330 keys (5 complete tiles and 10 tokens)
    hook.governor = None
    q1 = q[:, :, -1:]
    nc_np = np64(nc.cache)
    probe = O.hook_decode(np64(q1), np64(k), np64(v), nc_np, G, tau=-1.0)
    hook.tau = _gap_tau(probe["qn"][:, :, None].astype(np.float64) * nc_np[None, :, :T] / (64 * d))
    print(f"hook decode {dtype} tau={hook.tau}", flush=True)
    out1 = hook.orthocache_attention(q1, k, v, G)
    ref1 = O.hook_decode(np64(q1), np64(k), np64(v), nc_np, G, hook.tau)
    assert out1.shape == (B, Hq, 1, d)
    assert_out(out1, ref1["out"], dtype, f"hook decode {dtype}")
    assert 0 < ref1["skipped"].sum() < B * Hkv * T
    assert hook.stats['decode_steps'] == B
    assert hook.stats['decode_tiles_skipped'] == int(ref1["skipped"].sum())
    assert hook.stats['decode_tiles_total'] == B * Hkv * T
    np.testing.assert_allclose(hook.stats['hallucination_scores'][B:], ref1["h_score"], rtol=1e-5)
    assert hook.stats['layers_processed'] == 2


def test_hook_entropy_governor_and_short_context():
    from orthocache_gpu.model_hook import EntropyGovernor, OrthoCache_GQA_Attention
    B, Hq, Hkv, d, S = 2, 4, 2, 128, 150
    q, k, v = _qkv(B, Hq, Hkv, S, S, d, "f32", seed=12)
    gov = EntropyGovernor(alpha=0.5, beta=1.0, h_median=1.56)
    hook = OrthoCache_GQA_Attention(tau=-1.0, governor=gov)
    hook.orthocache_attention(q, k, v, 2)
    ref = O.hook_prefill(np64(q), np64(k), np64(v), 2, -1.0)
    np.testing.assert_allclose(gov.current_entropy, ref["entropy"][-1], rtol=1e-5)
    np.testing.assert_allclose(hook.stats['entropy'], ref["entropy"][-1], rtol=1e-5)
    assert hook.norm_cache is None and hook.stats['evicted_tiles'] == 0
    # under 64 keys: dense causal attention, no statistics
    qs, ks, vs = _qkv(1, 4, 2, 40, 40, 64, "bf16", seed=13)
    out = OrthoCache_GQA_Attention(tau=1.0).orthocache_attention(qs, ks, vs, 2)
    ref_s, _ = O.hook_causal_attention(np64(qs), np64(ks), np64(vs), 2)
    assert_out(out, ref_s, "bf16", "hook short context")


def test_hf_llama_patched_matches_dense():
    transformers = pytest.importorskip("transformers")
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention, patch_model_attention
    from orthocache_gpu.norm_cache import SpectralNormCache
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    model = transformers.LlamaForCausalLM(cfg).to(DEV).eval()
    ids = torch.randint(0, 128, (2, 104), generator=torch.Generator().manual_seed(1)).to(DEV)

    def run():
        with torch.no_grad():
            o = model(ids[:, :100], use_cache=True)
            logits, past = [o.logits[:, -1]], o.past_key_values
            for s in range(100, 104):
                o = model(ids[:, s:s + 1], past_key_values=past, use_cache=True)
                logits.append(o.logits[:, -1])
                past = o.past_key_values
        return torch.stack(logits)

    want = run()
    hook = OrthoCache_GQA_Attention(tau=-1.0)  # nothing is evicted: the hook must equal dense attention
    hook.norm_cache = SpectralNormCache(2, 8, torch.device(DEV))
    patch_model_attention(model, hook)
    got = run()
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)
    assert hook.stats['layers_processed'] == 2 * 5
    assert hook.stats['decode_steps'] == 2 * 2 * 4 and hook.stats['decode_tiles_skipped'] == 0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_hook_decode_scores_new_tiles_and_whole_tiles(dtype):
    """score_new_tiles=True (extension): tiles completed after the prefill are
    scored from the call's own K before the gate reads them; a context of whole
    tiles (no partial last tile) decodes like the oracle."""
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention
    from orthocache_gpu.norm_cache import SpectralNormCache
    B, Hq, Hkv, d, S0, S1 = 1, 4, 2, 128, 192, 384  # prefill 3 tiles, decode over 6
    G = Hq // Hkv
    q, k, v = _qkv(B, Hq, Hkv, S0, S1, d, dtype, seed=21)
    hook = OrthoCache_GQA_Attention(tau=-1.0, score_new_tiles=True)
    hook.norm_cache = SpectralNormCache(Hkv, 8, torch.device(DEV))
    hook.orthocache_attention(q, k[:, :, :S0], v[:, :, :S0], G)
    q1 = q[:, :, -1:]
    nc_before = np64(hook.norm_cache.cache).copy()
    want_norms = O.hook_tile_norms(np64(k))[0]  # (Hkv, 6)
    np.testing.assert_allclose(nc_before[:, :3], want_norms[:, :3], rtol=4 * 2.0 ** -23)
    assert not nc_before[:, 3:].any()
    probe = O.hook_decode(np64(q1), np64(k), np64(v), want_norms, G, tau=-1.0)
    hook.tau = _gap_tau(probe["qn"][:, :, None].astype(np.float64) * want_norms[None] / (64 * d))
    out = hook.orthocache_attention(q1, k, v, G)
    np.testing.assert_allclose(np64(hook.norm_cache.cache[:, :6]), want_norms, rtol=4 * 2.0 ** -23)
    ref = O.hook_decode(np64(q1), np64(k), np64(v), want_norms, G, hook.tau)
    assert_out(out, ref["out"], dtype, f"hook decode after append {dtype}")
    assert hook.stats['decode_tiles_skipped'] == int(ref["skipped"].sum())
    assert 0 < ref["skipped"].sum() < Hkv * 6


def test_group_gate_compares_in_float64():
    """The hook compares (qn * kn) / (64 d) <= tau in Python floats
    (perplexity_eval.py:480-491, :639-645): qn = kn = 1 + 2^-23 has the exact
    product 1 + 2^-22 + 2^-46, which float32 rounds down to 1 + 2^-22.  At
    tau_norm = 1 + 2^-22 the reference keeps the tile (a float32 compare
    would evict it); half of it is evicted either way."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    x = float(np.float32(1 + 2.0 ** -23))
    qn = torch.tensor([[x]], dtype=torch.float32, device=DEV)             # (batch 1, 1 kv head x G 1)
    kn = torch.tensor([[[x, x / 2]]], dtype=torch.float32, device=DEV)    # (1, 1 kv head, 2 tiles)
    assert (x * x) / 8192.0 > (1 + 2.0 ** -22) / 8192.0                   # the reference's compare
    for reduce in (N.OC_GROUP_MAX, N.OC_GROUP_MEDIAN):
        mask, _ = X.group_gate(qn, kn, 1, 1, 2, 2, 1 + 2.0 ** -22, reduce)
        assert mask.cpu().tolist() == [[[0, 1]]]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("B,Hq,Hkv,d,S", [(2, 8, 2, 128, 333), (1, 16, 2, 64, 320), (3, 4, 4, 128, 65),
                                         (1, 32, 8, 128, 4096)],
                         ids=lambda x: str(x))
def test_hook_decode_entry_point(dtype, B, Hq, Hkv, d, S):
    """oc_hook_decode (one call: q Walsh-subspace norms, group medians, gate,
    decode; one launch for 16-bit types, where the gate runs in the decode's
    prologue, two for float32) against the oracle's decode branch and against
    the same step composed from oc_row_norms, oc_group_gate and oc_decode:
    gate decisions and counts identical, outputs within the bar.  K is a slice of a longer cache and q
    the transposed view a decoder layer passes; S = 65 leaves one complete
    tile and a one-token tail."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    G = Hq // Hkv
    q, k, v = _qkv(B, Hq, Hkv, 1, S, d, dtype, seed=31 + S)
    T = S // 64
    g = torch.Generator().manual_seed(7)
    norms = (torch.rand((Hkv, T + 3), generator=g) * 40 + 1).to(DEV)  # a norm cache with spare columns
    probe = O.hook_decode(np64(q), np64(k), np64(v), np64(norms), G, tau=-1.0)
    tau = _gap_tau(probe["qn"][:, :, None].astype(np.float64) * np64(norms)[None, :, :T] / (64 * d)) if T > 1 else 0.5
    print(f"hook_decode entry {dtype} B={B} Hq={Hq} Hkv={Hkv} d={d} S={S} tau={tau}", flush=True)
    out, stats = X.hook_decode(q, k, v, norms, G, tau * 64 * d, 8)
    ref = O.hook_decode(np64(q), np64(k), np64(v), np64(norms), G, tau)
    assert out.shape == (B, Hq, 1, d) and out.dtype == TD[dtype]
    assert_out(out, ref["out"], dtype, f"oc_hook_decode {dtype} B={B} G={G} d={d} S={S}")
    st = stats.view(B, Hkv, 3).cpu().numpy()
    assert st[:, :, 0].sum(axis=1).tolist() == ref["skipped"].tolist()
    np.testing.assert_allclose(st[:, :, 1], ref["qn"], rtol=8 * 2.0 ** -23)
    # the composed path: the same kernels one by one
    qh = X.row_norms(q, low_band=8).view(B, Hq)
    keep, _, dev = X.group_gate(qh, norms[:Hkv].unsqueeze(0), Hkv, G, T, (S + 63) // 64, tau * 64 * d,
                                N.OC_GROUP_MEDIAN, keep_polarity=True, want_stats=True)
    # counts and tile norms exact; the group norm to float32 rounding (the
    # one-launch path sums q's squares in another order)
    dev = dev.view(B * Hkv, 3)
    assert torch.equal(dev[:, 0], stats[:, 0]) and torch.equal(dev[:, 2], stats[:, 2])
    torch.testing.assert_close(dev[:, 1], stats[:, 1], rtol=4 * 2.0 ** -23, atol=0)
    kv = X.rows_layout(k.reshape(B * Hkv, S, d), v.reshape(B * Hkv, S, d), partial_tail=True)
    res = X.decode(kv, q.reshape(B * Hq, d), G, gate=N.OC_GATE_MASK, threshold=0.0, mode=N.OC_MODE_CACHED,
                   out_dtype=q.dtype, tile_mask=keep.view(B * Hkv, -1))
    assert_out(out.view(B * Hq, d), np64(res.out), dtype, f"oc_hook_decode vs composed {dtype}", ref_rounded=True)


@pytest.mark.parametrize("qd,kd", [("bf16", "f32"), ("f16", "f32"), ("f32", "bf16"), ("bf16", "f16")])
def test_hook_decode_mixed_dtypes(qd, kd):
    """A cache whose type differs from the query's: the reference decodes
    from query.float(), key.float(), value.float() (perplexity_eval.py:
    590-592) and rounds once to the query's type.  oc_hook_decode widens
    every operand to float32 (exact) and rounds the output once, so the
    result equals the oracle on the float32 values of the stored operands
    within the query type's bar, and equals the all-float32 call rounded."""
    from orthocache_gpu import _launch as X
    B, Hq, Hkv, d, S = 2, 8, 2, 128, 333
    G = Hq // Hkv
    q, _, _ = _qkv(B, Hq, Hkv, 1, S, d, qd, seed=51)
    _, k, v = _qkv(B, Hq, Hkv, 1, S, d, kd, seed=52)
    T = S // 64
    g = torch.Generator().manual_seed(9)
    norms = (torch.rand((Hkv, T), generator=g) * 40 + 1).to(DEV)
    probe = O.hook_decode(np64(q), np64(k), np64(v), np64(norms), G, tau=-1.0)
    tau = _gap_tau(probe["qn"][:, :, None].astype(np.float64) * np64(norms)[None, :, :T] / (64 * d))
    print(f"hook_decode mixed q {qd} kv {kd}", flush=True)
    out, stats = X.hook_decode(q, k, v, norms, G, tau * 64 * d, 8)
    assert out.dtype == TD[qd]
    ref = O.hook_decode(np64(q), np64(k), np64(v), np64(norms), G, tau)
    assert_out(out, ref["out"], qd, f"oc_hook_decode mixed q {qd} kv {kd}")
    assert stats.view(B, Hkv, 3)[:, :, 0].sum(dim=1).cpu().tolist() == ref["skipped"].tolist()
    o32, _ = X.hook_decode(q.float(), k.float(), v.float(), norms, G, tau * 64 * d, 8)
    assert torch.equal(out, o32.to(TD[qd]))
