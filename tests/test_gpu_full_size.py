"""GPU parity at the BASELINE.json configurations as stated.

* The literal tau = 1.0 of configs 2, 3 and 4 at reduced size against the
  oracle.  The reference gate evicts a tile iff max_g ||q_g|| *
  ||(W K)[32:64]||_F <= tau with the full query norm
  (gqa_eviction.py:222-239); with N(0, 1) queries (||q|| ~ 11) every tile's
  bound is far above 1, so nothing is evicted.  Masks must be bit-exact and
  all-retained; outputs must meet the north-star bar.
* bench.py's primary step (batch 8, 64 kv rows, the library's default
  splits per workgroup: the exact parameter blocks the bench times), and
  configs 2 (batch 8, 65536 tokens), 3 (16 paged sequences of 4K..128K
  tokens) and 4 (fp8, batch 4, 131072 tokens, G = 8) at full size.  The
  properties checked hold at any size:
  - with a calibrated tau the mask equals the generator's tile labels;
  - with tau = 1.0 nothing is evicted;
  - the cached and single-pass decodes agree;
  - the output equals a float64 softmax over the retained tokens.
* Configs 0 (v1, one head, 4096 tokens, float32) and 1 (v2, 32 heads,
  float16, 1K / 4K / 32K tokens, bench.py's own parameter blocks) at their
  stated sizes against the oracle: masks bit-exact, outputs within the bar.
* The stand-alone oc_lse_merge against the oracle's sequential merge
  (fused_eviction.py:316-373) and against the decode's fused merge.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O
from tests.bars import assert_out

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield
    torch.cuda.empty_cache()


def np32(t):
    return t.detach().float().cpu().numpy()


def softmax_ref(q, k, v, keep_tiles, G, lengths=None, k_scales=None, v_scales=None, chunk=8):
    """float64 attention of every query head over the retained tokens of
    its kv row, on the GPU: q (rows * G, d), k / v (rows, S, d) (fp8 tensors
    decoded and multiplied by their per-tile scale in float32, as the
    decode defines the value), keep_tiles (rows, T) bool, lengths (rows,)
    token counts or None.  Rows with no retained token give zeros."""
    rows, s_len, d = k.shape
    out = torch.zeros((rows * G, d), dtype=torch.float64, device=DEV)
    tok = torch.arange(s_len, device=DEV)
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        kk, vv = k[r0:r1].float(), v[r0:r1].float()
        if k_scales is not None:
            kk = kk * k_scales[r0:r1].float().repeat_interleave(64, dim=1)[:, :s_len, None]
        if v_scales is not None:
            vv = vv * v_scales[r0:r1].float().repeat_interleave(64, dim=1)[:, :s_len, None]
        kk, vv = kk.double(), vv.double()
        qq = q[r0 * G:r1 * G].double().view(r1 - r0, G, d)
        logits = torch.bmm(qq, kk.transpose(1, 2).contiguous()) / math.sqrt(d)
        m = keep_tiles[r0:r1].repeat_interleave(64, dim=1)[:, :s_len]
        if lengths is not None:
            m = m & (tok[None, :] < lengths[r0:r1, None])
        logits = logits.masked_fill(~m[:, None, :], float("-inf"))
        p = torch.softmax(logits, dim=-1).nan_to_num(0.0)
        out[r0 * G:r1 * G] = torch.bmm(p, vv).reshape((r1 - r0) * G, d)
        del kk, vv, logits, p
    return out.cpu().numpy()


# ---------------------------------------------------------------- literal tau = 1.0


@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_config2_literal_tau1_vs_oracle(mode):
    """Config 2's recipe at reduced size (batch 2 x 2 kv heads, 12 tiles),
    two of each group's four query heads with no high head_dim band."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import make_kv, make_q
    G = 4
    wl = make_kv(4, 12 * 64, 128, noise_frac=0.5, dtype=torch.bfloat16, seed=21)
    q = make_q(4, G, 128, dtype=torch.bfloat16, seed=22, low_band_heads=2)
    sc = score_tiles(wl.keys.to(DEV))
    out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 1.0, G, mode=mode,
                                               score_cache=sc)
    ref, rmeta, rmask = O.gqa_v3(np32(q), np32(wl.keys), np32(wl.values), 1.0, G)
    assert rmask.all() and rmeta["tiles_evicted"] == 0
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask)
    assert m["tiles_evicted"] == 0 and m["eviction_rate"] == 0.0
    assert_out(out, ref, "bf16", f"config 2 tau=1 {mode}")


@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_config3_literal_tau1_vs_oracle(mode):
    """Config 3's recipe at reduced size: 3 sequences x 2 kv heads, G = 4,
    lengths 4096 / 1216 / 2560 tokens, 16-token pages in a shuffled pool,
    40% noise tiles."""
    from orthocache_gpu import fused_orthocache_attention_paged, score_paged_tiles
    from orthocache_gpu.workloads import make_kv, make_q, paged_pool
    B, hkv, G, d = 3, 2, 4, 128
    lens = [4096, 1216, 2560]
    wl = make_kv(B * hkv, 4096, d, noise_frac=0.4, dtype=torch.bfloat16, seed=31)
    kc, vc, bt = paged_pool(wl.keys, wl.values, hkv, 16, lens, seed=32)
    q = make_q(B * hkv, G, d, dtype=torch.bfloat16, seed=33)
    lt = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sc = score_paged_tiles(kc.to(DEV), bt.to(DEV), context_lens=lt)
    out, m = fused_orthocache_attention_paged(q.view(B, hkv * G, d).to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                              5.0, num_query_groups=G, tau=1.0, context_lens=lt, mode=mode,
                                              score_cache=sc)
    row_lens = [lens[r // hkv] for r in range(B * hkv)]
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate="cs", threshold=1.0, G=G, lengths=row_lens)
    live = sum(n // 64 for n in row_lens)
    assert ref["evicted"] == 0 and ref["retained"] == live
    assert m["tiles_evicted"] == 0 and m["tiles_retained"] == live
    assert_out(out.view(B * hkv * G, d), ref["out"], "bf16", f"config 3 tau=1 {mode}")


@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_config4_literal_tau1_vs_oracle(mode):
    """Config 4's recipe at reduced size: fp8-e4m3 K and V with one scale per
    (row, tile), G = 8, 2 rows of 12 tiles; scoring on the dequantised
    values."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import make_kv, make_q
    G = 8
    wl = make_kv(2, 12 * 64, 128, noise_frac=0.5, dtype=torch.float8_e4m3fn, seed=41)
    q = make_q(2, G, 128, dtype=torch.bfloat16, seed=42)
    ks, vs = wl.k_scales.to(DEV), wl.v_scales.to(DEV)
    sc = score_tiles(wl.keys.to(DEV), k_scale=ks)
    out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 1.0, G,
                                               k_scale=ks, v_scale=vs, mode=mode, score_cache=sc)
    tab = O.fp8_e4m3fn_table()
    kf = tab[wl.keys.view(torch.uint8).numpy()]
    vf = tab[wl.values.view(torch.uint8).numpy()]
    ref = O.decode_rows(np32(q), kf, vf, gate="cs", threshold=1.0, G=G, k_scales=wl.k_scales.numpy(),
                        v_scales=wl.v_scales.numpy())
    assert ref["keep"].all()
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), ref["keep"])
    assert_out(out, ref["out"], "fp8", f"config 4 tau=1 {mode}")


# ---------------------------------------------------------------- full size


def test_bench_primary_step_batch8():
    """bench.py's primary measurement: batch 8 (64 kv rows x 512 tiles, G =
    4), the bench's own parameter blocks (default splits per workgroup,
    merge fused, partials in the workspace), buffer set 0."""
    import bench
    st = bench.Setup(8)
    try:
        assert st.check() == 0.5  # the mask equals the generator's labels
        s0 = st.sets[0]
        outs = {}
        for variant in ("cached", "single_pass", "dense"):
            st.run(variant, 0)
            torch.cuda.synchronize()
            outs[variant] = st.out.clone()
        noise = s0["wl"].noise
        ref = softmax_ref(s0["q"], s0["wl"].keys, s0["wl"].values, noise, bench.G)
        assert_out(outs["cached"], ref, "bf16", "bench batch 8 cached")
        assert_out(outs["single_pass"], ref, "bf16", "bench batch 8 single pass")
        dense = softmax_ref(s0["q"], s0["wl"].keys, s0["wl"].values, torch.ones_like(noise), bench.G)
        assert_out(outs["dense"], dense, "bf16", "bench batch 8 dense")
        # and the secondary line's batch 1 (8 rows, 32 workgroups per row)
    finally:
        del st
        torch.cuda.empty_cache()


def test_bench_batch1_step():
    import bench
    st = bench.Setup(1, seed=100)
    try:
        assert st.check() == 0.5
        s0 = st.sets[0]
        st.run("cached", 0)
        torch.cuda.synchronize()
        ref = softmax_ref(s0["q"], s0["wl"].keys, s0["wl"].values, s0["wl"].noise, bench.G)
        assert_out(st.out, ref, "bf16", "bench batch 1 cached")
    finally:
        del st
        torch.cuda.empty_cache()


@pytest.mark.parametrize("recipe", ["tokens", "literal"])
@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_config0_full_size_vs_oracle(recipe, mode):
    """Config 0 as stated: v1 on q (1, 128) and K, V (4096, 128) float32,
    seed 0, zeta_max 5.0 (fused_eviction.py:698-800, CPU body :460-549).
    `tokens` builds the half-smooth / half-noise tiles along the token axis
    (the reference benchmark's construction), `literal` with the Walsh rows
    along head_dim (the config text read literally).  Mask bit-exact with
    the oracle, output within the float32 bar."""
    from orthocache_gpu import fused_orthocache_attention, score_tiles
    from orthocache_gpu.workloads import make_kv, make_kv_literal, make_q
    if recipe == "tokens":
        wl = make_kv(1, 4096, 128, noise_frac=0.5, dtype=torch.float32, seed=0)
        k, v = wl.keys[0], wl.values[0]
    else:
        k, _ = make_kv_literal(1, 4096, 128, dtype=torch.float32, seed=0)
        k = k[0]
        v = torch.randn((4096, 128), generator=torch.Generator().manual_seed(1))
    q = make_q(1, 1, 128, dtype=torch.float32, seed=2)
    ref, rmeta = O.fused_v1(np32(q), np32(k), np32(v), 5.0, return_mask=True)
    kd, vd = k.to(DEV), v.to(DEV)
    sc = score_tiles(kd.unsqueeze(0)) if mode == "cached" else None
    out, meta = fused_orthocache_attention(q.to(DEV), kd, vd, 5.0, return_mask=True, mode=mode, score_cache=sc)
    assert np.array_equal(meta["eviction_mask"].cpu().numpy(), rmeta["eviction_mask"]), recipe
    assert meta["tiles_retained"] == rmeta["tiles_retained"] and meta["tiles_evicted"] == rmeta["tiles_evicted"]
    if recipe == "tokens":
        assert rmeta["tiles_evicted"] == 32  # half of the 64 tiles are noise
    assert_out(out, ref, "f32", f"config 0 full size {recipe} {mode}")


@pytest.mark.parametrize("seq_len", [1024, 4096, 32768])
def test_config1_full_size_vs_oracle(seq_len):
    """Config 1 as stated and as bench.py times it (its Sweep parameter
    blocks, buffer set 0): v2, 32 heads, float16 q/K/V, zeta_max 5.0, over
    1K, 4K and 32K tokens (fused_eviction.py:573-691, CPU body :380-457).
    Dense, single-pass and cached decodes: masks bit-exact with the oracle,
    outputs within the float16 bar."""
    import bench
    sw = bench.Sweep(seq_len)
    try:
        s0 = sw.sets[0]
        q, k, v = s0["q"], s0["wl"].keys, s0["wl"].values
        print(f"config 1 full size S={seq_len}: oracle", flush=True)
        ref, rmeta, rmask = O.fused_v2(np32(q), np32(k), np32(v), 5.0)
        assert np.array_equal(rmask, ~s0["wl"].noise.cpu().numpy())
        for variant in ("single_pass", "cached"):
            rc = sw.lib.oc_decode(ctypes.byref(sw.params[variant][0]), ctypes.c_void_p(sw.stream))
            assert rc == 0
            torch.cuda.synchronize()
            assert_out(sw.out, ref, "f16", f"config 1 full size S={seq_len} {variant} (bench parameters)")
        # the drop-in API on the same inputs: its eviction mask
        from orthocache_gpu import fused_orthocache_attention_v2
        out, meta = fused_orthocache_attention_v2(q, k, v, 5.0)
        assert np.array_equal(meta["eviction_mask"].cpu().numpy(), rmask)
        assert meta["tiles_evicted"] == rmeta["tiles_evicted"]
        assert_out(out, ref, "f16", f"config 1 full size S={seq_len} v2 API")
        rc = sw.lib.oc_decode(ctypes.byref(sw.params["dense"][0]), ctypes.c_void_p(sw.stream))
        assert rc == 0
        torch.cuda.synchronize()
        dense = O.dense_decode(np32(q), np32(k), np32(v))
        assert_out(sw.out, dense, "f16", f"config 1 full size S={seq_len} dense (bench parameters)")
    finally:
        del sw
        torch.cuda.empty_cache()


def test_config2_full_size():
    """Batch 8 x 8 kv heads x 65536 tokens, bf16, G = 4 (two low-band query
    heads per group): calibrated tau (cached and single pass) and the
    literal tau = 1.0 (cached)."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q
    rows, G, S = 64, 4, 65536
    print("config 2 full size", flush=True)
    wl = make_kv(rows, S, 128, noise_frac=0.5, dtype=torch.bfloat16, device=DEV, seed=700)
    q = make_q(rows, G, 128, dtype=torch.bfloat16, device=DEV, seed=701, low_band_heads=2)
    sc = score_tiles(wl.keys)
    tau = calibrate_tau(sc.e_high, q, G)
    ref = softmax_ref(q, wl.keys, wl.values, wl.noise, G)
    for mode in ("cached", "single_pass"):
        out, m = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, tau, G, mode=mode, score_cache=sc)
        assert torch.equal(m["eviction_mask"], wl.noise), mode
        assert m["eviction_rate"] == 0.5
        assert_out(out, ref, "bf16", f"config 2 full size {mode}")
    out, m = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, 1.0, G, mode="cached", score_cache=sc)
    assert bool(m["eviction_mask"].all()) and m["tiles_evicted"] == 0
    dense = softmax_ref(q, wl.keys, wl.values, torch.ones_like(wl.noise), G)
    assert_out(out, dense, "bf16", "config 2 full size tau=1")


def test_config3_full_size():
    """16 sequences x 8 kv heads, lengths 4K..128K (bench.py's draw), 16-token
    pages in a shuffled pool, 40% noise tiles, G = 4: calibrated tau
    (cached, single pass) and tau = 1.0, through the decode call the bench
    times (flat workgroup layout, merge fused)."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q, paged_pool
    B, hkv, G, bs, s_max, seed = 16, 8, 4, 16, 131072, 300
    g = torch.Generator().manual_seed(seed)
    lens = (torch.randint(4096, s_max + 1, (B,), generator=g) // 64 * 64).tolist()
    print(f"config 3 full size, lengths {lens}", flush=True)
    wl = make_kv(B * hkv, s_max, 128, noise_frac=0.4, dtype=torch.bfloat16, device=DEV, seed=seed)
    kc, vc, bt = paged_pool(wl.keys, wl.values, hkv, bs, lens, seed=seed + 1)
    lt = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sc = score_paged_tiles(kc, bt, context_lens=lt)
    kv = X.paged_layout(kc, vc, bt, s_max // 64)
    kv.lengths = lt
    q = make_q(B * hkv, G, 128, dtype=torch.bfloat16, device=DEV, seed=seed + 2)
    row_len = torch.tensor([n for n in lens for _ in range(hkv)], device=DEV)
    live = torch.arange(s_max // 64, device=DEV)[None, :] < (row_len // 64)[:, None]
    tau = calibrate_tau(sc.e_high, q, G, live=live)
    want = wl.noise & live
    ref = softmax_ref(q, wl.keys, wl.values, want, G, lengths=row_len)
    for mode in (N.OC_MODE_CACHED, N.OC_MODE_SINGLE_PASS):
        res = X.decode(kv, q, G, gate=N.OC_GATE_CS, threshold=tau, mode=mode, scores=(sc.e_low, sc.e_high),
                       out_dtype=torch.bfloat16, want_keep=True)
        torch.cuda.synchronize()
        assert torch.equal(res.keep.bool() & live, want), f"mode {mode}"
        assert_out(res.out, ref, "bf16", f"config 3 full size mode {mode}")
    res = X.decode(kv, q, G, gate=N.OC_GATE_CS, threshold=1.0, mode=N.OC_MODE_CACHED, scores=(sc.e_low, sc.e_high),
                   out_dtype=torch.bfloat16, want_keep=True)
    torch.cuda.synchronize()
    assert torch.equal(res.keep.bool() & live, live)
    dense = softmax_ref(q, wl.keys, wl.values, live, G, lengths=row_len)
    assert_out(res.out, dense, "bf16", "config 3 full size tau=1")


def test_config4_full_size():
    """Batch 4 x 8 kv heads x 131072 tokens, fp8-e4m3 K and V with per-tile
    scales, G = 8: calibrated tau (cached, single pass) and tau = 1.0."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q
    rows, G, S, seed = 32, 8, 131072, 300
    print("config 4 full size", flush=True)
    wl = make_kv(rows, S, 128, noise_frac=0.5, dtype=torch.float8_e4m3fn, device=DEV, seed=seed)
    q = make_q(rows, G, 128, dtype=torch.bfloat16, device=DEV, seed=seed + 2)
    sc = score_tiles(wl.keys, k_scale=wl.k_scales)
    tau = calibrate_tau(sc.e_high, q, G)
    ref = softmax_ref(q, wl.keys, wl.values, wl.noise, G, k_scales=wl.k_scales, v_scales=wl.v_scales)
    for mode in ("cached", "single_pass"):
        out, m = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, tau, G, k_scale=wl.k_scales,
                                                   v_scale=wl.v_scales, mode=mode, score_cache=sc)
        assert torch.equal(m["eviction_mask"], wl.noise), mode
        assert_out(out, ref, "fp8", f"config 4 full size {mode}")
    out, m = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, 1.0, G, k_scale=wl.k_scales,
                                               v_scale=wl.v_scales, mode="cached", score_cache=sc)
    assert bool(m["eviction_mask"].all())
    dense = softmax_ref(q, wl.keys, wl.values, torch.ones_like(wl.noise), G, k_scales=wl.k_scales,
                        v_scales=wl.v_scales)
    assert_out(out, dense, "fp8", "config 4 full size tau=1")


# ---------------------------------------------------------------- stand-alone merge


@pytest.mark.parametrize("rows,P,d,out_dtype", [(5, 1, 128, torch.float32), (6, 7, 64, torch.bfloat16),
                                                 (4, 300, 128, torch.float16), (3, 8192, 64, torch.float32),
                                                 (2, 129, 128, torch.bfloat16)])
def test_lse_merge_standalone_vs_oracle(rows, P, d, out_dtype):
    """Synthetic partials: logit maxima spread over +-30, empty splits
    (m = -1e9, l = 0, acc = 0, as the decode writes them), one row with
    every split empty (-> zeros)."""
    from orthocache_gpu import _launch as X
    rng = np.random.default_rng(P * 7 + d)
    m = rng.uniform(-30, 30, (rows, P)).astype(np.float32)
    l = rng.uniform(0.5, 60.0, (rows, P)).astype(np.float32)
    acc = (rng.standard_normal((rows, P, d)) * l[..., None]).astype(np.float32)
    empty = rng.random((rows, P)) < 0.2
    empty[-1] = True
    m[empty], l[empty] = np.float32(-1e9), 0.0
    acc[empty] = 0.0
    got = X.lse_merge(torch.from_numpy(m).to(DEV), torch.from_numpy(l).to(DEV), torch.from_numpy(acc).to(DEV),
                      out_dtype=out_dtype)
    bar = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[out_dtype]
    # the merge in exact arithmetic (float64): sum_s e^(m_s - M) acc_s / max(sum_s e^(m_s - M) l_s, 1e-9)
    w = np.exp(m.astype(np.float64) - m.max(axis=1, keepdims=True))
    exact = (w[..., None] * acc).sum(axis=1) / np.maximum((w * l).sum(axis=1), 1e-9)[:, None]
    assert_out(got, exact, bar, f"lse_merge rows={rows} P={P} d={d} vs exact")
    if out_dtype != torch.float32:
        # the same merge before the output's 16-bit rounding: float32 out
        # against exact arithmetic at the float32 bar, so that the 16-bit
        # figure above is the output rounding alone
        got32 = X.lse_merge(torch.from_numpy(m).to(DEV), torch.from_numpy(l).to(DEV), torch.from_numpy(acc).to(DEV),
                            out_dtype=torch.float32)
        assert_out(got32, exact, "f32", f"lse_merge rows={rows} P={P} d={d} vs exact, before {bar} rounding")
    if P <= 512:
        # the oracle's sequential float32 merge accumulates one rounding per
        # split; over thousands of splits that alone nears the float32 bar
        ref = np.stack([O.lse_merge(m[r], l[r], acc[r]) for r in range(rows)])
        assert not ref[-1].any()
        assert_out(got, ref, bar, f"lse_merge rows={rows} P={P} d={d} vs oracle")
    assert not got[-1].any()


@pytest.mark.parametrize("gate", ["cs", "zeta"])
def test_lse_merge_of_decode_partials(gate):
    """oc_decode with out = NULL returns one partial per logical split (the
    sequence-split multi-GPU path); oc_lse_merge of them equals the fused
    merge of the same call and the oracle."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import make_kv, make_q
    G = 4 if gate == "cs" else 1
    wl = make_kv(3, 40 * 64, 128, dtype=torch.bfloat16, device=DEV, seed=9)
    q = make_q(3, G, 128, dtype=torch.bfloat16, device=DEV, seed=10)
    kv = X.rows_layout(wl.keys, wl.values)
    thr = 150.0 if gate == "cs" else 5.0
    gcode = N.OC_GATE_CS if gate == "cs" else N.OC_GATE_ZETA
    res = X.decode(kv, q, G, gate=gcode, threshold=thr, num_splits=11, out_dtype=torch.float32, want_partials=True)
    merged = X.lse_merge(*res.partials, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_out(merged, np32(res.out), "f32", f"lse_merge vs fused merge {gate}")
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G, num_splits=11)
    assert_out(merged, ref["out"], "f32", f"lse_merge of partials vs oracle {gate}")
