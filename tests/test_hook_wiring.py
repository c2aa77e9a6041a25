"""CPU tests of the model hook's host logic: patch_model_attention routes
every decoder layer >= min_layer of a transformers Llama model through the
hook with (batch, heads, seq, head_dim) tensors (a tiny random-init model;
the hook's attention is replaced by torch's SDPA here, since the kernels
need the GPU), and the governors follow the reference's formulas."""

import math

import pytest
import torch

transformers = pytest.importorskip("transformers")


def _tiny_llama(layers=3):
    cfg = transformers.LlamaConfig(vocab_size=96, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return transformers.LlamaForCausalLM(cfg).eval()


def test_patch_routes_sdpa_through_hook():
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention, patch_model_attention
    model = _tiny_llama()
    ids = torch.randint(0, 96, (2, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = model(ids).logits
    hook = OrthoCache_GQA_Attention(tau=0.5)
    seen = []
    sdpa = torch.nn.functional.scaled_dot_product_attention  # the patch swaps the module attribute

    def fake(query, key, value, num_query_groups):
        seen.append((tuple(query.shape), tuple(key.shape), num_query_groups))
        return sdpa(query, key, value, is_causal=query.shape[2] > 1, enable_gqa=True)

    hook.orthocache_attention = fake
    patch_model_attention(model, hook, min_layer=1)
    with torch.no_grad():
        got = model(ids).logits
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert seen == [((2, 4, 40, 32), (2, 2, 40, 32), 2)] * 2  # layers 1 and 2 only
    # the module-level SDPA is restored after each layer
    assert torch.nn.functional.scaled_dot_product_attention is sdpa


def test_governors():
    from oracle import orthocache_oracle as O
    from orthocache_gpu.model_hook import EntropyGovernor, ResidualGovernor
    g = ResidualGovernor(alpha=0.5)
    for r in (0.2, 0.3):
        g.report_layer(r)
    assert g.get_tau_effective(2.0) == O.residual_tau(2.0, 0.5, [0.2, 0.3])
    assert g.layer_history == [0.2, 0.3]
    g.reset()
    assert g.eps_accum == 0.0 and g.get_tau_effective(2.0) == 2.0
    e = EntropyGovernor(alpha=0.5, beta=2.0, h_median=1.0)
    assert e.get_tau_effective(1.0) == 1.0
    e.report_layer(0.4)
    e.set_entropy(1.5)
    assert math.isclose(e.get_tau_effective(1.0), O.entropy_tau(1.0, 0.5, [0.4], 2.0, 1.0, 1.5), rel_tol=1e-15)


def test_hook_stats_shape():
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention
    h = OrthoCache_GQA_Attention(tau=2.0)
    assert h.eviction_rate == 0.0 and h.norm_cache is None
    assert set(h.stats) == {'total_tiles', 'evicted_tiles', 'layers_processed', 'cs_bounds',
                            'hallucination_scores', 'q_search_intensity', 'k_info_density', 'decode_steps',
                            'decode_tiles_skipped', 'decode_tiles_total'}
    h.stats['total_tiles'], h.stats['evicted_tiles'] = 10, 4
    assert h.eviction_rate == 0.4
    h.reset_stats()
    assert h.stats['total_tiles'] == 0


def test_hook_fails_loudly_on_cpu_tensors():
    from orthocache_gpu.model_hook import OrthoCache_GQA_Attention
    q = torch.randn(1, 4, 70, 64)
    k = torch.randn(1, 2, 70, 64)
    with pytest.raises((RuntimeError, ValueError)):
        OrthoCache_GQA_Attention(tau=1.0).orthocache_attention(q, k, k, 2)


def test_stats_fold_lazily_in_call_order():
    """Per-call values wait on the device and are folded, in order, by the
    first read of the dict (one transfer)."""
    from orthocache_gpu.model_hook import _empty_stats
    st = _empty_stats()
    seen = []

    def make(i):
        def fold(host):
            seen.append((i, host.tolist()))
            st['layers_processed'] += 1
        return fold
    for i in range(3):
        st.defer(make(i), torch.tensor([float(i), 2.0 * i]))
    assert seen == []
    assert st['layers_processed'] == 3
    assert seen == [(0, [0.0, 0.0]), (1, [1.0, 2.0]), (2, [2.0, 4.0])]
    for i in range(300):  # the pending list is bounded
        st.defer(make(i), torch.tensor([1.0]))
    assert len(st._pending) < 256
    assert dict.__getitem__(st, 'layers_processed') >= 3 + 256


def test_decode_stats_fold_together_as_one_by_one():
    """Runs of decode calls of one shape fold in one numpy pass; the lists and
    counters equal those of folding each call alone (NaN, negative and zero
    norms included), and a call of another shape or kind ends the run."""
    import numpy as np
    from orthocache_gpu.model_hook import _decode_folds, _empty_stats
    rng = np.random.default_rng(3)
    B, Hkv, T = 2, 4, 9
    devs = []
    for i in range(7):
        x = rng.standard_normal((B, Hkv, 3)).astype(np.float32)
        x[..., 0] = rng.integers(0, T + 1, (B, Hkv))
        if i == 2:
            x[1, 2, 1] = np.nan
        if i == 4:
            x[0, :, 2] = -1.0
        devs.append(torch.from_numpy(x))
    one, many = _empty_stats(), _empty_stats()
    other = torch.zeros((B, Hkv + 1, 3))
    order = list(range(4)) + ["other"] + list(range(4, 7))
    for st, batched in ((one, False), (many, True)):
        for i in order:
            if i == "other":
                f, fm = _decode_folds(st, None, B, Hkv + 1, T)
                st.defer(f, other, (("decode", B, Hkv + 1, T), fm) if batched else None)
                continue
            f, fm = _decode_folds(st, None, B, Hkv, T)
            st.defer(f, devs[i], (("decode", B, Hkv, T), fm) if batched else None)
    a, b = dict(one.items()), dict(many.items())
    for key in a:
        if isinstance(a[key], list):
            assert len(a[key]) == len(b[key]) and all(
                (x == y) or (x != x and y != y) for x, y in zip(a[key], b[key])), key
            assert all(type(y) is float for y in b[key]), key
        else:
            assert a[key] == b[key], key
    assert a['decode_steps'] == 8 * B and a['layers_processed'] == 8


def test_stats_ring_rows_reused_after_fold():
    """A decode call's statistics rows come from a ring of _MAX_PENDING rows
    per shape; a fold frees them, and rows taken without a deferred call (a
    call that failed) never run past the ring."""
    from orthocache_gpu.model_hook import _empty_stats
    st = _empty_stats()
    n = st._MAX_PENDING
    rows = [st.ring_rows(torch.device("cpu"), (2, 2, 3)) for _ in range(3)]
    assert all(r.shape == (2, 2, 3) and r.is_contiguous() for r in rows)
    assert rows[0].data_ptr() != rows[1].data_ptr()
    st.defer(lambda h: None, rows[0])
    _ = st['layers_processed']  # a read folds: the ring starts over
    assert st.ring_rows(torch.device("cpu"), (2, 2, 3)).data_ptr() == rows[0].data_ptr()
    for _ in range(3 * n):  # rows taken, nothing deferred
        st.ring_rows(torch.device("cpu"), (2, 2, 3))
