"""GPU parity: the HIP path (through liborthocache_hip's C ABI) against the
oracle and the reference's golden vectors.

Bars: eviction masks, tile assignment and counts
bit-exact; outputs within 1e-5 (fp32), 2e-3 (fp16/bf16), 2e-2 (fp8 inputs)
max-abs against the unrounded oracle, plus half an output ulp for the
output's own rounding (tests/bars.py; a golden vector is itself rounded,
so against it the slack is one ulp).
"""

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O
from tests import golden_io
from tests.bars import assert_out

pytestmark = pytest.mark.gpu

DEV = "cuda"
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield


def np32(t):
    return t.detach().float().cpu().numpy()


def to_dev(raw, dt):
    """golden raw array -> device tensor of the stored dtype"""
    if dt == "f32":
        return torch.from_numpy(raw.astype(np.float32)).to(DEV)
    if dt in ("f16", "bf16"):
        return torch.from_numpy(raw.astype(np.uint16).view(np.int16)).view(TORCH_DT[dt]).to(DEV)
    if dt == "fp8":
        return torch.from_numpy(raw.astype(np.uint8)).view(torch.float8_e4m3fn).to(DEV)
    if dt == "i32":
        return torch.from_numpy(raw.astype(np.int32)).to(DEV)
    raise ValueError(dt)


# ---------------------------------------------------------------- library

def test_library_and_device():
    import orthocache_gpu._native as N
    assert "gfx950" in N.version()
    props = torch.cuda.get_device_properties(0)
    assert N.device_cu_count() == props.multi_processor_count


def test_fp8_decode_is_exact():
    """fwht of a tile whose only non-zero token is token 0 gives k0/8 in every
    spectral row, so row 0 of the transform reads back the decoded fp8 codes."""
    from orthocache_gpu import fwht_tiles
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    k = torch.zeros((2 * 64, 128), dtype=torch.uint8)
    k[0] = codes[:128]
    k[64] = codes[128:]
    x = fwht_tiles(k.view(torch.float8_e4m3fn).to(DEV))
    got = np.concatenate([np32(x[0, 0]), np32(x[1, 0])]) * 8.0
    ref = O.fp8_e4m3fn_table()
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


# ---------------------------------------------------------------- scores / FWHT

def test_golden_scores_bit_exact_mask():
    from orthocache_gpu import triton_fwht_eviction
    raw, dec, dt, meta, params, _ = golden_io.load("fwht_scores")
    keys = to_dev(raw["keys"], "f32")
    mask, zeta = triton_fwht_eviction(keys, params["zeta_max"], return_zeta=True)
    assert np.array_equal(mask.cpu().numpy(), dec["mask"].astype(bool))
    np.testing.assert_allclose(np32(zeta), dec["zeta"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [64, 128])
def test_integer_tiles_scores_exact(dtype, d):
    """Integer tiles in [-4, 4]: exact in every summation order, so e_low,
    e_high and zeta must equal the float64 closed forms bit for bit."""
    from orthocache_gpu import score_tiles
    rng = np.random.default_rng(d)
    k = rng.integers(-4, 5, size=(3, 8 * 64, d)).astype(np.float32)
    sc = score_tiles(torch.from_numpy(k).to(TORCH_DT[dtype]).to(DEV), zeta_max=1.0)
    for r in range(3):
        for t in range(8):
            kt = k[r, t * 64:(t + 1) * 64].astype(np.float64)
            eh = 0.5 * np.sum((kt[:32] - kt[32:]) ** 2)
            s_r = np.stack([kt[i::8].sum(axis=0) for i in range(8)])
            el = np.sum(s_r ** 2) / 8.0 - np.sum(kt.sum(axis=0) ** 2) / 64.0
            assert float(sc.e_high[r, t]) == eh
            assert float(sc.e_low[r, t]) == el
            z = np.float32(np.float32(eh) / np.float32(np.float32(el) + np.float32(1e-6)))
            assert float(sc.zeta[r, t]) == float(z)
            assert bool(sc.keep[r, t]) == (not float(z) > 1.0)


def test_fwht_full_transform():
    from orthocache_gpu import fwht_tiles
    rng = np.random.default_rng(4)
    k = rng.standard_normal((5 * 64, 128)).astype(np.float32)
    x = np32(fwht_tiles(torch.from_numpy(k).to(DEV)))
    w = O.walsh_matrix().astype(np.float64)
    for t in range(5):
        ref = w @ k[t * 64:(t + 1) * 64].astype(np.float64)
        np.testing.assert_allclose(x[t], ref, atol=2e-5)
        np.testing.assert_allclose(x[t], O.fwht64_butterfly(k[t * 64:(t + 1) * 64]), atol=2e-5)


# ---------------------------------------------------------------- golden cases

@pytest.mark.parametrize("name", ["v1_f32", "v1_fp8k_bf16q"])
def test_golden_v1(name):
    from orthocache_gpu import fused_orthocache_attention
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention(to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]),
                                        to_dev(raw["values"], dt["values"]), params["zeta_max"],
                                        return_mask=True, k_scale=params.get("k_scale", 1.0))
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), meta["eviction_mask"])
    for k in ("tiles_retained", "tiles_evicted", "eviction_rate"):
        assert m[k] == meta[k]
    bar = "fp8" if dt["keys"] == "fp8" else dt["out"]
    assert_out(out, dec["out"], bar, name, ref_rounded=True)


@pytest.mark.parametrize("name", ["v2_f32", "v2_f16", "v2_bf16"])
def test_golden_v2(name):
    from orthocache_gpu import fused_orthocache_attention_v2
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_v2(to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]),
                                           to_dev(raw["values"], dt["values"]), params["zeta_max"])
    for k, v in meta.items():
        assert m[k] == v, k
    assert m["tile_assignment"] == "interleaved"
    assert_out(out, dec["out"], dt["out"], name, ref_rounded=True)


@pytest.mark.parametrize("name", ["v3_f32", "v3_bf16", "v3_fp8k"])
def test_golden_v3(name):
    from orthocache_gpu import fused_orthocache_attention_v3_gqa
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_v3_gqa(
        to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]), to_dev(raw["values"], dt["values"]),
        params["tau"], params["G"], k_scale=params.get("k_scale", 1.0))
    for k, v in meta.items():
        assert m[k] == v, k
    bar = "fp8" if dt["keys"] == "fp8" else dt["out"]
    assert_out(out, dec["out"], bar, name, ref_rounded=True)


@pytest.mark.parametrize("name", ["paged_bs16", "paged_bs32", "paged_fp8k"])
def test_golden_paged(name):
    from orthocache_gpu import fused_orthocache_attention_paged
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_paged(
        to_dev(raw["q"], dt["q"]), to_dev(raw["k_cache"], dt["k_cache"]), to_dev(raw["v_cache"], dt["v_cache"]),
        to_dev(raw["block_tables"], "i32"), params["zeta_max"], k_scale=params.get("k_scale", 1.0))
    assert m["layout"] == "paged"
    bar = "fp8" if dt["k_cache"] == "fp8" else dt["out"]
    assert_out(out, dec["out"], bar, name, ref_rounded=True)


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("gate", ["zeta", "cs"])
@pytest.mark.parametrize("lens", [False, True])
@pytest.mark.parametrize("vdt", ["bf16", "fp8"])
def test_paged_fp8_k_in_kernel(bs, G, gate, lens, vdt, monkeypatch):
    """fp8 K with a scalar k_scale and bf16 q, cached-score decode: the
    scoring and the decode kernels round float(k) * k_scale to bf16 as they
    widen K (OC_KSCALE_DEQUANT), the reference's k_cache.to(q.dtype) *
    k_scale (paged_eviction.py:354-357), and a bf16 V beside the fp8 K is read
    as it is: no copy of either pool.  The scores equal, bit for bit, those of
    the pool dequantised beforehand; masks, counts and outputs match the
    oracle on the dequantised values, as the copy path's do."""
    from orthocache_gpu import fused_orthocache_attention_paged
    from orthocache_gpu import _launch as X
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_q, paged_pool
    B, hkv, tiles, d = 2, 2, 6, 128
    ks = 0.37  # not a power of two: the rounding after the product matters
    wl = _mixed(B * hkv, tiles, d, "f32", seed=bs + G)
    k8 = (wl.keys / ks).to(torch.float8_e4m3fn)
    kd = (k8.float() * ks).to(torch.bfloat16)  # the reference's dequantised K
    vv = wl.values.to(TORCH_DT[vdt])
    seq_lens = [tiles * 64 - 70, tiles * 64] if lens else [tiles * 64] * B
    k8c, vc, bt = paged_pool(k8, vv, hkv, bs, seq_lens, seed=7)
    kdc, _, _ = paged_pool(kd, vv, hkv, bs, seq_lens, seed=7)
    k8c, vc, bt, kdc = k8c.to(DEV), vc.to(DEV), bt.to(DEV), kdc.to(DEV)
    assert torch.equal(X.dequant_fp8(k8c, ks, torch.bfloat16), kdc)
    q = make_q(B * hkv, G, d, seed=bs).to(DEV)
    cl = torch.tensor(seq_lens, dtype=torch.int32, device=DEV) if lens else None
    sc = score_paged_tiles(k8c, bt, k_scale=ks, q_dtype=torch.bfloat16, context_lens=cl)
    sc_ref = score_paged_tiles(kdc, bt, context_lens=cl)
    assert torch.equal(sc.e_low, sc_ref.e_low) and torch.equal(sc.e_high, sc_ref.e_high)
    row_lens = [seq_lens[r // hkv] for r in range(B * hkv)]
    live = (torch.arange(tiles, device=DEV)[None, :] * 64 + 64
            <= torch.tensor(row_lens, device=DEV)[:, None]) if lens else None
    thr = calibrate_tau(sc_ref.e_high, q, G, live) if gate == "cs" else 5.0
    kw = dict(num_query_groups=G, mode="cached", context_lens=cl)
    if gate == "cs":
        kw["tau"] = thr
    if not lens:
        kw["num_splits"] = 256  # whole rows over many splits, several per workgroup
    qb = q.view(B, hkv * G, d)
    ref = O.decode_rows(np32(q), np32(kd), np32(vv), gate=gate, threshold=thr, G=G, lengths=row_lens)
    out_copy, mc = fused_orthocache_attention_paged(qb, kdc, vc, bt, 5.0, k_scale=1.0, score_cache=sc_ref, **kw)
    # the in-kernel path: no dequantised copy of K, no conversion of V
    monkeypatch.setattr(X, "dequant_fp8", lambda *a, **k: pytest.fail("the K pool was dequantised"))
    real_harmonize = X.harmonize_kv
    monkeypatch.setattr(X, "harmonize_kv", lambda k, v: real_harmonize(k, v) if v is None or v.dtype == k.dtype
                        else pytest.fail("K or V was converted"))
    out, m = fused_orthocache_attention_paged(qb, k8c, vc, bt, 5.0, k_scale=ks, score_cache=sc, **kw)
    for mm in (m, mc):
        assert mm["tiles_retained"] == ref["retained"] and mm["tiles_evicted"] == ref["evicted"]
    assert 0 < ref["retained"] and 0 < ref["evicted"]
    what = f"paged fp8 K in-kernel bs={bs} G={G} {gate} lens={lens} V={vdt}"
    assert_out(out.view(-1, d), ref["out"], "bf16", what)
    assert_out(out_copy.view(-1, d), ref["out"], "bf16", what + " (copy path)")


def test_paged_fp8_k_beside_f16_v_dequantises_the_pool():
    """fp8 K with a scalar k_scale beside a V of neither K's type nor bf16
    (float16), bf16 q, cached decode: the wrapper dequantises the pool, as
    the reference does, instead of asking for the in-kernel form."""
    from orthocache_gpu import fused_orthocache_attention_paged
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    from orthocache_gpu.workloads import make_q, paged_pool
    B, hkv, tiles, d, bs, ks = 2, 2, 4, 128, 16, 0.37
    wl = _mixed(B * hkv, tiles, d, "f32", seed=11)
    k8 = (wl.keys / ks).to(torch.float8_e4m3fn)
    kd = (k8.float() * ks).to(torch.bfloat16)
    vv = wl.values.to(torch.float16)
    k8c, vc, bt = paged_pool(k8, vv, hkv, bs, [tiles * 64] * B, seed=2)
    k8c, vc, bt = k8c.to(DEV), vc.to(DEV), bt.to(DEV)
    q = make_q(B * hkv, 1, d, seed=3).to(DEV)
    sc = score_paged_tiles(k8c, bt, k_scale=ks, q_dtype=torch.bfloat16)
    out, m = fused_orthocache_attention_paged(q.view(B, hkv, d), k8c, vc, bt, 5.0, k_scale=ks, mode="cached",
                                              score_cache=sc)
    ref = O.decode_rows(np32(q), np32(kd), np32(vv), gate="zeta", threshold=5.0, G=1)
    assert m["tiles_retained"] == ref["retained"]
    assert_out(out.view(-1, d), ref["out"], "bf16", "paged fp8 K beside f16 V")


# ---------------------------------------------------------------- random vs oracle

def _mixed(rows, tiles, d, dtype, seed, noise_frac=0.5):
    from orthocache_gpu.workloads import make_kv
    return make_kv(rows, tiles * 64, d, noise_frac=noise_frac, dtype=TORCH_DT[dtype], seed=seed)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("num_splits", [None, 1, 3, 7, 40])
def test_v2_random_vs_oracle(dtype, d, num_splits):
    from orthocache_gpu import fused_orthocache_attention_v2
    wl = _mixed(3, 21, d, dtype, seed=5)
    q = torch.randn((3, d), generator=torch.Generator().manual_seed(2)).to(TORCH_DT[dtype])
    out, m = fused_orthocache_attention_v2(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 5.0,
                                           num_splits=num_splits)
    ref, rmeta, rmask = O.fused_v2(np32(q), np32(wl.keys), np32(wl.values), 5.0)
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask)
    assert np.array_equal(rmask, ~wl.noise.numpy())
    for k in ("tiles_retained", "tiles_evicted", "eviction_rate"):
        assert m[k] == rmeta[k]
    assert_out(out, ref, dtype, "v2")


# head_dim 128 over every group size and both 16-bit types; head_dim 64 on a
# reduced grid (bf16, G in 1/4/8)
_V3_GRID = [(G, mode, dtype, 128) for G in (1, 2, 3, 4, 5, 8, 12) for mode in ("single_pass", "cached")
            for dtype in ("bf16", "f16")]
_V3_GRID += [(G, mode, "bf16", 64) for G in (1, 4, 8) for mode in ("single_pass", "cached")]


@pytest.mark.parametrize("G,mode,dtype,d", _V3_GRID)
def test_v3_random_vs_oracle(G, mode, dtype, d):
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_q
    tdt = TORCH_DT[dtype]
    wl = _mixed(2, 17, d, dtype, seed=G)
    q = make_q(2, G, d, dtype=tdt, seed=G + 1, low_band_heads=min(2, G))
    sc = score_tiles(wl.keys.to(DEV))
    tau = calibrate_tau(sc.e_high, q.to(DEV), G)
    out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), tau, G,
                                               mode=mode, score_cache=sc)
    ref, rmeta, rmask = O.gqa_v3(np32(q), np32(wl.keys), np32(wl.values), tau, G)
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask)
    assert np.array_equal(rmask, wl.noise.numpy())  # CS keeps the noise tiles
    for k in ("tiles_retained", "tiles_evicted", "eviction_rate", "num_kv_heads", "num_query_groups",
              "gate_type"):
        assert m[k] == rmeta[k]
    assert_out(out, ref, dtype, f"v3 G={G} {mode} {dtype} d={d}")


@pytest.mark.parametrize("gate", ["none", "zeta", "cs"])
@pytest.mark.parametrize("P", [1, 2, 5, 16])
def test_split_partials_and_assignment(gate, P):
    """The partial state of split s covers exactly tiles {s + kP}: compare
    every (m, l, acc) partial with the oracle's per-split online softmax."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa
    G = 2
    wl = _mixed(2, 13, 64, "f32", seed=P)
    q = torch.randn((4, 64), generator=torch.Generator().manual_seed(P))
    thr = {"none": 0.0, "zeta": 5.0, "cs": 150.0}[gate]
    if gate == "cs":
        out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), thr, G,
                                                   num_splits=P, return_partials=True)
    else:
        import orthocache_gpu._launch as X
        import orthocache_gpu._native as N
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
        res = X.decode(kv, q.to(DEV), G, gate={"none": N.OC_GATE_NONE, "zeta": N.OC_GATE_ZETA}[gate],
                       threshold=thr, num_splits=P, out_dtype=torch.float32, want_keep=True,
                       want_partials=True)
        torch.cuda.synchronize()
        m = {"partials": res.partials}
        out = res.out
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G,
                        num_splits=P, want_partials=True)
    pm, pl, pacc = (np32(x) for x in m["partials"])
    assert np.array_equal(pm == np.float32(-1e9), ref["M"] == np.float32(-1e9))  # same empty splits
    np.testing.assert_allclose(pm, ref["M"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pl, ref["L"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(pacc, ref["ACC"], rtol=1e-5, atol=1e-5)
    assert_out(out, ref["out"], "f32", "merged")


def test_fused_merge_counters_and_fallback():
    """The split merge runs in the last decode workgroup of each row (merge
    counters in the workspace) unless Pg > 4 * head_dim, where the separate
    merge kernel runs.  Calls of different shapes in a row, on both paths,
    must all match the oracle and leave the counters zero."""
    import orthocache_gpu._launch as X
    import orthocache_gpu._native as N
    cases = [(3, 40, 128, 40, 1), (2, 9, 128, None, 0), (1, 300, 64, 300, 1), (3, 40, 128, 7, 0),
             (1, 300, 64, 300, 1), (2, 9, 128, 3, 2)]
    for i, (rows, tiles, d, P, spw) in enumerate(cases):
        wl = _mixed(rows, tiles, d, "f32", seed=30 + i)
        q = torch.randn((rows * 2, d), generator=torch.Generator().manual_seed(i))
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
        res = X.decode(kv, q.to(DEV), 2, gate=N.OC_GATE_CS, threshold=150.0, num_splits=P,
                       out_dtype=torch.float32, splits_per_group=spw)
        torch.cuda.synchronize()
        ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate="cs", threshold=150.0, G=2,
                            num_splits=res.num_splits)
        assert_out(res.out, ref["out"], "f32", f"case {i}")
    # same shape, new data each call: the merge must read this call's partials
    for i in range(4):
        wl = _mixed(2, 24, 128, "bf16", seed=50 + i)
        q = torch.randn((8, 128), generator=torch.Generator().manual_seed(60 + i)).to(torch.bfloat16)
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
        res = X.decode(kv, q.to(DEV), 4, gate=N.OC_GATE_CS, threshold=150.0, num_splits=24,
                       out_dtype=torch.float32, splits_per_group=2)
        torch.cuda.synchronize()
        ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate="cs", threshold=150.0, G=4,
                            num_splits=24)
        assert_out(res.out, ref["out"], "f32", f"repeat {i}")
    for buf in X._WORKSPACES.values():
        assert int(buf[: 64 << 10].count_nonzero()) == 0, "merge counters not left zero"


@pytest.mark.parametrize("tiles", [45, 160])
@pytest.mark.parametrize("spw", [2, 3, 8, 64])
@pytest.mark.parametrize("gate", ["cs", "zeta"])
def test_balanced_cached_decode(spw, gate, tiles):
    """Cached mode with several splits per workgroup: the workgroups of a row
    take equal shares of the row's retained tiles by rank, or (with at least
    32 tiles per workgroup) take ranks from a shared counter.  The output, the
    keep mask and the retained counts must match the oracle, with context
    lengths that cut tiles (partial tail tiles are always retained)."""
    import orthocache_gpu._launch as X
    import orthocache_gpu._native as N
    from orthocache_gpu.workloads import calibrate_tau, make_q
    G = 4
    wl = _mixed(3, tiles, 128, "bf16", seed=40 + spw)
    q = make_q(3, G, 128, dtype=torch.bfloat16, seed=spw, low_band_heads=2)
    lens = torch.tensor([tiles * 64, 1000, 64 * 7], dtype=torch.int32)
    kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
    kv.lengths = lens.to(DEV)
    el, eh, _, _ = X.score_tiles(kv, want_zeta=False, want_keep=False)
    if gate == "cs":
        thr = calibrate_tau(eh, q.to(DEV), G)
        gcode = N.OC_GATE_CS
    else:
        thr, gcode = 5.0, N.OC_GATE_ZETA
    for P in (None, 9):
        res = X.decode(kv, q.to(DEV), G, gate=gcode, threshold=thr, mode=N.OC_MODE_CACHED, scores=(el, eh),
                       num_splits=P, out_dtype=torch.float32, want_keep=True, splits_per_group=spw)
        torch.cuda.synchronize()
        ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G,
                            lengths=lens.tolist(), num_splits=res.num_splits)
        got_keep = res.keep.cpu().numpy().astype(bool)
        for r, n in enumerate(lens.tolist()):
            nt = (n + 63) // 64
            assert np.array_equal(got_keep[r, :nt], ref["keep"][r, :nt]), f"row {r}"
        assert_out(res.out, ref["out"], "f32", f"balanced spw={spw} P={P}")
    for buf in X._WORKSPACES.values():
        assert int(buf[: 64 << 10].count_nonzero()) == 0, "counters not left zero"


def test_v1_matches_oracle_and_reference_edge_cases():
    from orthocache_gpu import fused_orthocache_attention
    g = torch.Generator().manual_seed(42)
    q = torch.randn(1, 128, generator=g)
    k = torch.randn(8 * 64, 128, generator=g)
    v = torch.randn(8 * 64, 128, generator=g)
    # zero eviction == dense (test_fused_integration.py:59-104)
    out, m = fused_orthocache_attention(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=1e9, return_mask=True)
    assert m["tiles_evicted"] == 0 and m["tiles_retained"] == 8
    assert_out(out, O.dense_decode(np32(q), np32(k)[None], np32(v)[None]), "f32", "dense")
    # total eviction -> zeros, no NaN (test_fused_integration.py:290-306)
    out, m = fused_orthocache_attention(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=0.001, return_mask=True)
    assert m["tiles_retained"] == 0 and torch.all(out == 0)
    # large logits (x100), single tile
    out, _ = fused_orthocache_attention((q * 100).to(DEV), (k[:256] * 100).to(DEV), v[:256].to(DEV), 1e9)
    assert torch.isfinite(out).all()
    ref = O.dense_decode(np32(q * 100), np32(k[:256] * 100)[None], np32(v[:256])[None])
    assert_out(out, ref, "f32", "large logits")
    out, _ = fused_orthocache_attention(q.to(DEV), k[:64].to(DEV), v[:64].to(DEV), 1e9)
    assert torch.isfinite(out).all()


def test_v2_zeta_max_zero_and_many_splits():
    from orthocache_gpu import fused_orthocache_attention_v2
    g = torch.Generator().manual_seed(42)
    q = torch.randn(1, 128, generator=g)
    k = torch.randn(1, 512, 128, generator=g)
    v = torch.randn(1, 512, 128, generator=g)
    out, m = fused_orthocache_attention_v2(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=0.0, num_splits=4)
    assert out.shape == (1, 128) and torch.isfinite(out).all()
    out1, _ = fused_orthocache_attention_v2(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=1e6, num_splits=1)
    out16, m16 = fused_orthocache_attention_v2(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=1e6, num_splits=16)
    assert m16["num_splits"] == 16
    assert_out(out16, np32(out1), "f32", "1 vs 16 splits")
    assert_out(out1, O.dense_decode(np32(q), np32(k), np32(v)), "f32", "dense")


@pytest.mark.parametrize("gate", ["cs", "zeta"])
def test_single_pass_long_split_list(gate):
    """One split of 2100 tiles: more keep flags than the matrix-core single
    pass stages in LDS (2048), so they are stored from inside the tile loop.
    Mask = generator labels = oracle; output against the oracle."""
    from orthocache_gpu import fused_orthocache_attention_v2, fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_q
    wl = _mixed(1, 2100, 128, "bf16", seed=31)
    if gate == "cs":
        G = 4
        q = make_q(1, G, 128, dtype=torch.bfloat16, seed=32)
        tau = calibrate_tau(score_tiles(wl.keys.to(DEV)).e_high, q.to(DEV), G)
        out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), tau, G,
                                                   num_splits=1)
        ref, rmeta, rmask = O.gqa_v3(np32(q), np32(wl.keys), np32(wl.values), tau, G)
        want = wl.noise.numpy()
    else:
        q = torch.randn((1, 128), generator=torch.Generator().manual_seed(33)).to(torch.bfloat16)
        out, m = fused_orthocache_attention_v2(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 5.0, num_splits=1)
        ref, rmeta, rmask = O.fused_v2(np32(q), np32(wl.keys), np32(wl.values), 5.0)
        want = ~wl.noise.numpy()
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask)
    assert np.array_equal(rmask, want)
    assert m["tiles_retained"] == rmeta["tiles_retained"]
    assert_out(out, ref, "bf16", f"single split {gate}")


@pytest.mark.parametrize("tiles,gate", [(3000, "cs"), (16500, "cs"), (16500, "zeta")])
def test_cached_decode_long_rows(tiles, gate):
    """Cached decode of rows longer than the per-wave-prologue kernel takes
    (2048 tiles) and, at 16,500 tiles, longer than the in-LDS retained-tile
    bitmask of the balanced layout (16,384): the general kernel's paths for
    such rows, with a length that cuts the last tile.  Keep flags and output
    against the oracle."""
    import orthocache_gpu._launch as X
    import orthocache_gpu._native as N
    from orthocache_gpu.workloads import calibrate_tau, make_q
    G, d = 4, 64
    wl = _mixed(2, tiles, d, "bf16", seed=tiles + 1)
    q = make_q(2, G, d, dtype=torch.bfloat16, seed=tiles + 2)
    lens = torch.tensor([tiles * 64 - 5, 2100 * 64 + 10], dtype=torch.int32)
    kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
    kv.lengths = lens.to(DEV)
    el, eh, _, _ = X.score_tiles(kv, want_zeta=False, want_keep=False)
    if gate == "cs":
        thr, gcode = calibrate_tau(eh, q.to(DEV), G), N.OC_GATE_CS
    else:
        thr, gcode = 5.0, N.OC_GATE_ZETA
    res = X.decode(kv, q.to(DEV), G, gate=gcode, threshold=thr, mode=N.OC_MODE_CACHED, scores=(el, eh),
                   out_dtype=torch.float32, want_keep=True)
    torch.cuda.synchronize()
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G,
                        lengths=lens.tolist())
    got_keep = res.keep.cpu().numpy().astype(bool)
    for r, n in enumerate(lens.tolist()):
        nt = (n + 63) // 64
        assert np.array_equal(got_keep[r, :nt], ref["keep"][r, :nt]), f"row {r}"
    assert 0 < int(ref["keep"].sum()) < ref["keep"].size
    assert_out(res.out, ref["out"], "bf16", f"long rows {tiles} {gate}")


def test_auto_num_splits_on_device():
    from orthocache_gpu import fused_orthocache_attention_v2
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for tiles, want in ((4, 1), (128, 32), (512, min(cus, 128)), (2048, min(cus, 512))):
        q = torch.zeros(1, 64, device=DEV)
        k = torch.zeros(1, tiles * 64, 64, device=DEV)
        _, m = fused_orthocache_attention_v2(q, k, k, 5.0)
        assert m["num_splits"] == want == O.auto_num_splits(tiles, cus)


def test_context_lengths_vs_oracle():
    from orthocache_gpu import fused_orthocache_attention_v3_gqa
    wl = _mixed(3, 6, 128, "f32", seed=9)
    q = torch.randn((6, 128), generator=torch.Generator().manual_seed(3))
    lens = torch.tensor([150, 384, 1], dtype=torch.int32)
    out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 150.0, 2,
                                               context_lens=lens.to(DEV), num_splits=3)
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate="cs", threshold=150.0, G=2,
                        lengths=lens.tolist(), num_splits=3)
    assert_out(out, ref["out"], "f32", "lengths")
    assert m["tiles_retained"] == ref["retained"]
    assert m["tiles_evicted"] == ref["evicted"]


FLAT_CASES = [("cs", "cached", "bf16", 4, False), ("cs", "single_pass", "bf16", 4, False),
              ("zeta", "single_pass", "bf16", 1, False), ("zeta", "cached", "f32", 1, False),
              ("none", "single_pass", "bf16", 4, False), ("cs", "cached", "bf16", 12, False),
              ("cs", "single_pass", "f32", 2, False), ("cs", "cached", "bf16", 4, True),
              ("cs", "single_pass", "bf16", 4, True)]


@pytest.mark.parametrize("gate,mode,dtype,G,paged", FLAT_CASES)
def test_variable_lengths_flat_layout(gate, mode, dtype, G, paged):
    """Rows of very different lengths (one 700-tile row with a partial tail,
    a 3-tile row, a partial single tile, an empty row): the flat workgroup
    layout gives the long row many workgroups (up to the 512-per-row cap) and
    each short row one; outputs and masks against the oracle."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import calibrate_tau, make_q, paged_pool
    lens = [700 * 64 + 17, 3 * 64, 37, 0]
    rows, T, d = len(lens), 701, 128
    wl = _mixed(rows, T, d, dtype, seed=41)
    q = make_q(rows, G, d, dtype=TORCH_DT[dtype], seed=42)
    el, eh, _, _ = X.score_tiles(X.rows_layout(wl.keys.to(DEV), None))
    if paged:
        kc, vc, bt = paged_pool(wl.keys, wl.values, 1, 16, lens, seed=43)
        kv = X.paged_layout(kc.to(DEV), vc.to(DEV), bt.to(DEV), T)
    else:
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    gcode = {"none": N.OC_GATE_NONE, "zeta": N.OC_GATE_ZETA, "cs": N.OC_GATE_CS}[gate]
    thr = {"cs": calibrate_tau(eh, q.to(DEV), G) if gate == "cs" else 0.0, "zeta": 5.0, "none": 0.0}[gate]
    res = X.decode(kv, q.to(DEV), G, gate=gcode, threshold=thr,
                   mode=N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS, scores=(el, eh),
                   out_dtype=TORCH_DT[dtype], want_keep=True)
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G, lengths=lens)
    if gate != "none":
        assert np.array_equal(res.keep[:, :T].cpu().numpy().astype(bool), ref["keep"])
    assert_out(res.out, ref["out"], dtype, f"flat {gate} {mode} {dtype} G={G} paged={paged}")


MANY_ROW_CASES = [("cs", "cached", "bf16", 4, False), ("cs", "single_pass", "bf16", 4, False),
                  ("none", "single_pass", "bf16", 1, False), ("zeta", "cached", "f32", 2, False),
                  ("cs", "cached", "bf16", 4, True), ("cs", "single_pass", "bf16", 2, True)]


@pytest.mark.parametrize("gate,mode,dtype,G,paged", MANY_ROW_CASES)
def test_flat_layout_many_rows(gate, mode, dtype, G, paged):
    """2100 rows of random lengths (0..256 tokens, empty and partial-tile rows
    among them): more rows than a workgroup keeps in registers while it cuts
    the flat layout (1024 with 4-wave, 2048 with 8-wave workgroups), so the
    rows past those are read again in every pass; most rows get a single
    short share.  Outputs and masks against the oracle."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import calibrate_tau, make_q, paged_pool
    rows, T, d = 2100, 4, 64
    rng = np.random.default_rng(77)
    lens = rng.integers(0, T * 64 + 1, size=rows)
    lens[:40:3] = 0
    lens[1:60:4] = T * 64
    lens = [int(v) for v in lens]
    wl = _mixed(rows, T, d, dtype, seed=78)
    q = make_q(rows, G, d, dtype=TORCH_DT[dtype], seed=79)
    el, eh, _, _ = X.score_tiles(X.rows_layout(wl.keys.to(DEV), None))
    if paged:
        kc, vc, bt = paged_pool(wl.keys, wl.values, 1, 16, lens, seed=80)
        kv = X.paged_layout(kc.to(DEV), vc.to(DEV), bt.to(DEV), T)
    else:
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    gcode = {"none": N.OC_GATE_NONE, "zeta": N.OC_GATE_ZETA, "cs": N.OC_GATE_CS}[gate]
    thr = {"cs": calibrate_tau(eh, q.to(DEV), G) if gate == "cs" else 0.0, "zeta": 5.0, "none": 0.0}[gate]
    res = X.decode(kv, q.to(DEV), G, gate=gcode, threshold=thr,
                   mode=N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS, scores=(el, eh),
                   out_dtype=torch.float32, want_keep=True)
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate=gate, threshold=thr, G=G, lengths=lens)
    if gate != "none":
        assert np.array_equal(res.keep[:, :T].cpu().numpy().astype(bool), ref["keep"])
    # float32 output: the short rows' outputs are single V values (up to ~3.6),
    # where a 16-bit output's rounding alone would exceed the bar
    assert_out(res.out, ref["out"], dtype, f"many rows {gate} {mode} {dtype} G={G} paged={paged}")


@pytest.mark.parametrize("block_size", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("dtype,d", [("f32", 64), ("bf16", 128)])
def test_paged_equals_contiguous(block_size, dtype, d):
    """Shuffled physical pool == contiguous rows (test_paged_eviction.py:28-90).
    bf16 with pages of >= 16 tokens runs on the matrix-core path."""
    from orthocache_gpu import fused_orthocache_attention_paged, fused_orthocache_attention_v2
    from orthocache_gpu.workloads import paged_pool
    B, H = 2, 4
    wl = _mixed(B * H, 4, d, dtype, seed=block_size)
    q = torch.randn((B, H, d), generator=torch.Generator().manual_seed(1)).to(TORCH_DT[dtype])
    kc, vc, bt = paged_pool(wl.keys, wl.values, H, block_size, [256] * B, seed=3)
    out, m = fused_orthocache_attention_paged(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), 5.0)
    ref = torch.stack([fused_orthocache_attention_v2(q[b].to(DEV), wl.keys[b * H:(b + 1) * H].to(DEV),
                                                     wl.values[b * H:(b + 1) * H].to(DEV), 5.0)[0]
                       for b in range(B)])
    if dtype == "f32":
        torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    else:
        assert_out(out, np32(ref), dtype, "paged vs contiguous", ref_rounded=True)
    oref, _, omask = O.paged(np32(q), np32(kc), np32(vc), bt.numpy(), 5.0)
    assert_out(out, oref, dtype, "paged vs oracle")
    assert m["tiles_retained"] == int(omask.sum())


@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_paged_gqa_context_lens_cs(mode):
    """Extension: GQA + per-sequence lengths + CS gate on a 16-token page pool
    (config 3's recipe at small size)."""
    from orthocache_gpu import fused_orthocache_attention_paged, score_paged_tiles
    from orthocache_gpu.workloads import make_q, paged_pool
    B, Hkv, G, d, tiles = 3, 2, 4, 128, 9
    wl = _mixed(B * Hkv, tiles, d, "bf16", seed=21, noise_frac=0.4)
    lens = [576, 300, 64 * 5]
    kc, vc, bt = paged_pool(wl.keys, wl.values, Hkv, 16, lens, seed=4)
    q = make_q(B * Hkv, G, d, seed=5)
    sc = score_paged_tiles(kc.to(DEV), bt.to(DEV), context_lens=torch.tensor(lens).to(DEV))
    out, m = fused_orthocache_attention_paged(q.view(B, Hkv * G, d).to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                              5.0, num_query_groups=G, tau=150.0,
                                              context_lens=torch.tensor(lens, dtype=torch.int32).to(DEV),
                                              mode=mode, score_cache=sc)
    row_lens = [lens[r // Hkv] for r in range(B * Hkv)]
    ref = O.decode_rows(np32(q), np32(wl.keys), np32(wl.values), gate="cs", threshold=150.0, G=G,
                        lengths=row_lens)
    assert_out(out.view(B * Hkv * G, d), ref["out"], "bf16", "paged gqa")
    assert m["tiles_retained"] == ref["retained"] and m["tiles_evicted"] == ref["evicted"]


@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_fp8_tile_scales_vs_oracle(mode):
    """Extension (config 4's recipe at small size): fp8-e4m3fn K and V with
    one fp32 scale per (row, tile), G=8, CS gate."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import make_q
    G = 8
    wl = _mixed(2, 12, 128, "fp8", seed=8)
    q = make_q(2, G, 128, seed=6)
    sc = score_tiles(wl.keys.to(DEV), k_scale=wl.k_scales.to(DEV))
    out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), wl.keys.to(DEV), wl.values.to(DEV), 150.0, G,
                                               k_scale=wl.k_scales.to(DEV), v_scale=wl.v_scales.to(DEV),
                                               mode=mode, score_cache=sc)
    tab = O.fp8_e4m3fn_table()
    kf = tab[wl.keys.view(torch.uint8).numpy()]
    vf = tab[wl.values.view(torch.uint8).numpy()]
    ref = O.decode_rows(np32(q), kf, vf, gate="cs", threshold=150.0, G=G,
                        k_scales=wl.k_scales.numpy(), v_scales=wl.v_scales.numpy())
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), ref["keep"])
    assert_out(out, ref["out"], "fp8", "fp8 tiles")


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("gate,mode", [("cs", "single_pass"), ("cs", "cached"), ("zeta", "single_pass"),
                                       ("none", "single_pass")])
@pytest.mark.parametrize("paged", [False, True])
def test_fp8_tile_scales_grid(d, gate, mode, paged):
    """fp8-e4m3fn K and V with per-(row, tile) scales and bf16 q (the
    matrix-core path, K and V widened to bf16 exactly), contiguous and on a
    16-token page pool, with a partial tail tile; masks and outputs against
    the oracle on the decoded values."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import calibrate_tau, make_q, paged_pool
    G, rows, T = 4, 3, 13
    wl = _mixed(rows, T, d, "fp8", seed=50 + d)
    q = make_q(rows, G, d, seed=51)
    lens = [T * 64, T * 64 - 20, 5 * 64]
    tab = O.fp8_e4m3fn_table()
    kf = tab[wl.keys.view(torch.uint8).numpy()]
    vf = tab[wl.values.view(torch.uint8).numpy()]
    ks, vs = wl.k_scales.to(DEV), wl.v_scales.to(DEV)
    el, eh, _, _ = X.score_tiles(_with_kscales(X.rows_layout(wl.keys.to(DEV), None), ks))
    if paged:
        kc, vc, bt = paged_pool(wl.keys.view(torch.uint8), wl.values.view(torch.uint8), 1, 16, lens, seed=52)
        kv = X.paged_layout(kc.view(torch.float8_e4m3fn).to(DEV), vc.view(torch.float8_e4m3fn).to(DEV),
                            bt.to(DEV), T)
    else:
        kv = X.rows_layout(wl.keys.to(DEV), wl.values.to(DEV))
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    _with_kscales(kv, ks)
    kv.v_scale_mode, kv.v_scales = X.vscale_mode(vs, kv.num_rows, kv.num_tiles, DEV)
    gcode = {"none": N.OC_GATE_NONE, "zeta": N.OC_GATE_ZETA, "cs": N.OC_GATE_CS}[gate]
    thr = {"cs": calibrate_tau(eh, q.to(DEV), G) if gate == "cs" else 0.0, "zeta": 5.0, "none": 0.0}[gate]
    res = X.decode(kv, q.to(DEV), G, gate=gcode, threshold=thr,
                   mode=N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS, scores=(el, eh),
                   out_dtype=torch.bfloat16, want_keep=True)
    ref = O.decode_rows(np32(q), kf, vf, gate=gate, threshold=thr, G=G, lengths=lens,
                        k_scales=wl.k_scales.numpy(), v_scales=wl.v_scales.numpy())
    if gate != "none":
        assert np.array_equal(res.keep[:, :T].cpu().numpy().astype(bool), ref["keep"])
    assert_out(res.out, ref["out"], "fp8", f"fp8 d={d} {gate} {mode} paged={paged}")


def _with_kscales(kv, ks):
    from orthocache_gpu import _launch as X
    kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(ks, kv.num_rows, kv.num_tiles, ks.device)
    return kv


def test_orthocache_forward_modes():
    from orthocache_gpu import orthocache_forward
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2, 128, generator=g)
    k = torch.randn(512, 2, 128, generator=g)
    v = torch.randn(512, 2, 128, generator=g)
    out, meta = orthocache_forward(q.to(DEV), k.to(DEV), v.to(DEV), block_size=512, zeta_max=5.0,
                                   mode="triton_fused")
    assert out.shape == (1, 2, 128)
    assert "num_splits" in meta and meta["tile_assignment"] == "interleaved" and "latency_ms" in meta
    ref, _, _ = O.fused_v2(np32(q[0]), np32(k.permute(1, 0, 2)), np32(v.permute(1, 0, 2)), 5.0)
    assert_out(out[0], ref, "f32", "triton_fused")
    qd = torch.randn(3, 2, 128, generator=g)
    out, meta = orthocache_forward(qd.to(DEV), k.to(DEV), v.to(DEV), mode="dense")
    ref = np.stack([O.dense_decode(np32(qd[s]), np32(k.permute(1, 0, 2)), np32(v.permute(1, 0, 2)))
                    for s in range(3)])
    assert_out(out, ref, "f32", "dense")
    out, meta = orthocache_forward(q.to(DEV), k[:100].to(DEV), v[:100].to(DEV), mode="triton_fused",
                                   crossover_threshold=4096)
    assert meta["crossover_fallback"] and meta["actual_mode"] == "dense"
    ref = O.dense_decode(np32(q[0]), np32(k[:100].permute(1, 0, 2)), np32(v[:100].permute(1, 0, 2)))
    assert_out(out[0], ref, "f32", "crossover dense")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_paged_bad_block_id_rejected(dtype):
    from orthocache_gpu import fused_orthocache_attention_paged
    dt = TORCH_DT[dtype]
    q = torch.randn(1, 2, 64, device=DEV).to(dt)
    kc = torch.randn(4, 2, 32, 64, device=DEV).to(dt)
    bt = torch.tensor([[0, 7]], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="block id"):
        fused_orthocache_attention_paged(q, kc, kc, bt, 5.0)


@pytest.mark.parametrize("bs", [16, 32])
def test_paged_bad_block_id_rejected_matrix_core(bs):
    """The same check on the matrix-core path with the per-wave prologue
    (bf16, pages of >= 16 tokens, cached mode over rows of given lengths):
    an id outside the pool, in a tile past the first, reads as zeros and
    raises, and the valid table gives the oracle's output."""
    from orthocache_gpu import fused_orthocache_attention_paged
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    g = torch.Generator().manual_seed(5)
    hkv, G, d, nb = 2, 2, 64, 32
    blocks = 256 // bs
    q = torch.randn(1, hkv * G, d, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.randn(nb, hkv, bs, d, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(nb, hkv, bs, d, generator=g).to(torch.bfloat16).to(DEV)
    bt = torch.randperm(nb, generator=g)[:blocks].to(torch.int32).view(1, -1).to(DEV)
    lens = torch.tensor([250], dtype=torch.int32, device=DEV)
    sc = score_paged_tiles(kc, bt, context_lens=lens)
    out, _ = fused_orthocache_attention_paged(q, kc, vc, bt, 5.0, num_query_groups=G, tau=-1.0,
                                              context_lens=lens, mode="cached", score_cache=sc)
    k_rows = kc[bt[0].long()].permute(1, 0, 2, 3).reshape(hkv, -1, d)[:, :250]
    v_rows = vc[bt[0].long()].permute(1, 0, 2, 3).reshape(hkv, -1, d)[:, :250]
    ref = np.stack([O.dense_decode(np32(q[0, h * G:(h + 1) * G]), np.broadcast_to(np32(k_rows[h]), (G, 250, d)),
                                   np.broadcast_to(np32(v_rows[h]), (G, 250, d))) for h in range(hkv)])
    assert_out(out[0], ref.reshape(hkv * G, d), "bf16", f"paged matrix-core bs={bs}")
    bad = bt.clone()
    bad[0, blocks - 2] = nb + 7
    with pytest.raises(ValueError, match="block id"):
        fused_orthocache_attention_paged(q, kc, vc, bad, 5.0, num_query_groups=G, tau=-1.0, context_lens=lens,
                                         mode="cached", score_cache=sc)


# ---------------------------------------------------------------- full size properties

@pytest.mark.parametrize("gate", ["cs", "zeta"])
def test_headline_size_properties(gate):
    """At the headline shape (GQA 32/8, d=128, 32K tokens, bf16): the mask is
    exactly the generator's tile labels, cached == single-pass, and the
    output equals a float64 softmax over the retained tokens."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, fused_orthocache_attention_v2, score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q
    Hkv, G, S, d = 8, 4, 32768, 128
    wl = make_kv(Hkv, S, d, dtype=torch.bfloat16, device=DEV, seed=0)
    q = make_q(Hkv, G, d, device=DEV, seed=1)
    sc = score_tiles(wl.keys)
    if gate == "cs":
        tau = calibrate_tau(sc.e_high, q, G)
        o1, m1 = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, tau, G)
        o2, m2 = fused_orthocache_attention_v3_gqa(q, wl.keys, wl.values, tau, G, mode="cached", score_cache=sc)
        want = wl.noise
    else:
        qq = q.view(Hkv, G, d)[:, 0].contiguous()
        o1, m1 = fused_orthocache_attention_v2(qq, wl.keys, wl.values, 5.0)
        o2, m2 = fused_orthocache_attention_v2(qq, wl.keys, wl.values, 5.0, mode="cached", score_cache=sc)
        q, G, want = qq, 1, ~wl.noise
    assert torch.equal(m1["eviction_mask"], want)
    assert torch.equal(m2["eviction_mask"], want)
    assert m1["eviction_rate"] == 0.5
    assert (o1.float() - o2.float()).abs().max().item() <= 2e-3
    keep_tok = want.repeat_interleave(64, dim=1)  # (Hkv, S)
    k64, v64, q64 = wl.keys.double(), wl.values.double(), q.double().view(Hkv, G, d)
    logits = torch.einsum("hgd,hsd->hgs", q64, k64) / d ** 0.5
    logits = logits.masked_fill(~keep_tok[:, None, :], float("-inf"))
    ref = torch.einsum("hgs,hsd->hgd", torch.softmax(logits, dim=-1), v64).reshape(Hkv * G, d)
    assert_out(o1, ref.cpu().numpy(), "bf16", f"headline B=1 {gate} single pass")
    assert_out(o2, ref.cpu().numpy(), "bf16", f"headline B=1 {gate} cached")
