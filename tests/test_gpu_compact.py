"""GPU parity of orthocache_forward(mode='compact') and its 512-token
spectral pipeline against the oracle: oc_block_spectra (band energies,
zeta, AC and spatial energy, block mean, query-aware bounds), stream
compaction, the spectral_energy / adaptive_attention / perfect_eviction
functions and the whole compact forward (gates, metadata, output).

Bars: energies and bounds within 1e-5 relative (float32 sums against the
float64 oracle); masks and orders exact (data built with margins: smooth
blocks have zeta < 1, noise blocks zeta > 100, thresholds placed in gaps);
outputs (always bfloat16, as the reference returns) within 2e-3 plus half
a bfloat16 ulp.
"""

import math

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


_W = O.fwht512(np.eye(512))  # H512 / sqrt(512), symmetric


def _keys(nb, H, d, noise_blocks, seed, dtype):
    """Blocks W @ C: smooth (C on rows 1..4) or noise (C on rows 256..511,
    for every head of the blocks in noise_blocks), plus 0.05 white noise."""
    rng = np.random.default_rng(seed)
    k = np.zeros((nb * 512, H, d))
    for b in range(nb):
        for h in range(H):
            c = np.zeros((512, d))
            if b in noise_blocks:
                c[256:] = rng.standard_normal((256, d))
            else:
                c[1:5] = 4 * rng.standard_normal((4, d))
                c[0] = rng.standard_normal(d)
            k[512 * b:512 * (b + 1), h] = _W @ c + 0.05 * rng.standard_normal((512, d))
    return torch.from_numpy(k).to(TD[dtype])


# d = 96 and 40: the generic head_dim path, whose eight-column groups (12, 5)
# do not divide the 256 threads
_SPEC_GRID = [(dt, d) for dt in ("f32", "bf16", "f16") for d in (64, 128)] + [("bf16", 96), ("f32", 40)]


@pytest.mark.parametrize("dtype,d", _SPEC_GRID)
def test_block_spectra_vs_oracle(dtype, d):
    from orthocache_gpu import _launch as X
    k = _keys(5, 3, d, {1, 3}, seed=d, dtype=dtype)
    q = torch.randn((4, 3, d), generator=torch.Generator().manual_seed(1)).to(TD[dtype])
    kt = torch.cat([k, k[:100]]).to(DEV)  # 100 tokens past the last block are not read
    got = X.block_spectra(kt, q.to(DEV), want_bounds=True, want_mean=True)
    ref = O.block_spectra(np64(k), np64(q))
    for name in ("e_low", "e_mid", "e_high", "e_ac", "energy", "zeta", "max_bound"):
        np.testing.assert_allclose(np64(got[name]), ref[name], rtol=1e-5, atol=1e-6, err_msg=name)
    np.testing.assert_allclose(np64(got["block_mean"]), ref["block_mean"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(np64(got["bounds"]), ref["bounds"], rtol=1e-5, atol=1e-5)
    z = np64(got["zeta"])
    assert (z[[1, 3]] > 100).all() and (z[[0, 2, 4]] < 1).all()


def test_stream_compact_and_spectral_api():
    from orthocache_gpu import spectral_energy as SE
    from orthocache_gpu.adaptive_attention import stream_compact
    rng = np.random.default_rng(5)
    for n in (1, 5, 1500, 3000):
        m = rng.random(n) < 0.3
        idx, cnt = stream_compact(torch.from_numpy(m).to(DEV))
        ref_idx, ref_cnt = O.stream_compact(m)
        assert cnt == ref_cnt and np.array_equal(idx.cpu().numpy(), ref_idx)
    k = _keys(3, 2, 64, {2}, seed=6, dtype="f32")
    q = torch.randn((2, 2, 64), generator=torch.Generator().manual_seed(2))
    ref = O.block_spectra(np64(k), np64(q))
    kd, qd = k.to(DEV), q.to(DEV)
    dc, lo, mid, hi = SE.compute_spectral_bands(kd)
    np.testing.assert_allclose(np64(dc), ref["block_mean"] * math.sqrt(512), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np64(SE.compute_spectral_decay_ratio(kd)), ref["zeta"], rtol=1e-5)
    np.testing.assert_allclose(np64(SE.compute_block_energy(kd)), ref["energy"], rtol=1e-5)
    np.testing.assert_allclose(np64(SE.compute_query_aware_bounds(qd, kd)), ref["bounds"], rtol=1e-5, atol=1e-5)
    tau = float(np.median(ref["max_bound"]))
    assert np.array_equal(SE.compute_query_aware_mask(qd, kd, tau).cpu().numpy(), ref["max_bound"] >= tau)
    mm = SE.compute_multiband_mask(qd, kd, tau, 5.0).cpu().numpy()
    assert np.array_equal(mm, (ref["max_bound"] >= tau) & (ref["zeta"] <= 5.0))
    with pytest.raises(RuntimeError, match="invalid"):
        SE.compute_spectral_decay_ratio(kd[:700])
    with pytest.raises(NotImplementedError):
        SE.compute_spectral_bands(kd, band_low=(1, 32))


@pytest.mark.parametrize("nb,H", [(32, 64), (40, 64), (9, 300), (1, 5)])
def test_compact_gate_kernel_vs_oracle(nb, H):
    """oc_compact_gate on synthetic tables, with the (block, head) entries
    staged in LDS (nb * H <= 2048 and H <= 256) and read from global memory
    (2560 entries; 300 heads): masks, counts and regimes exact, statistics
    within 1e-5.  Data with margins: kept bounds in [200, 210], evicted in
    [0, 100] (tau = 150), zeta < 1 or > 100 (zeta_max = 5), evicted blocks'
    beta about 10 (perfect: gap ~ 195) or 150 (statistical: gap ~ 55)."""
    from orthocache_gpu import _launch as X
    rng = np.random.default_rng(nb * 1000 + H)
    d = 64
    kind = rng.integers(0, 3, nb)  # 0 kept, 1 evicted perfect, 2 evicted statistical
    kind[0] = 0
    mb = np.where(kind[:, None] == 0, rng.uniform(200, 210, (nb, H)), rng.uniform(0, 100, (nb, H)))
    zeta = np.where(rng.random((nb, H)) < 0.8, rng.uniform(0, 1, (nb, H)), rng.uniform(100, 1e4, (nb, H)))
    zeta[kind == 0, 0] = 0.5  # a kept block has a head that passes both gates
    beta = np.where(kind == 2, 150.0, 10.0)[:, None] * rng.uniform(0.9, 1.0, (nb, H))
    energy = (beta * math.sqrt(d)) ** 2  # beta = qmax * sqrt(E) / sqrt(d) with qmax = 1
    qmax = np.ones(H)
    spec = {"max_bound": torch.tensor(mb, dtype=torch.float32, device=DEV),
            "zeta": torch.tensor(zeta, dtype=torch.float32, device=DEV),
            "energy": torch.tensor(energy, dtype=torch.float32, device=DEV),
            "q_norm_max": torch.tensor(qmax, dtype=torch.float32, device=DEV)}
    f32 = lambda x: np.asarray(x, dtype=np.float32)
    for tau in (150.0, None):
        bm, tm, st = X.compact_gate(spec, d, tau, 5.0, O.F32_UNDERFLOW, 8)
        ref = O.compact_gate(f32(mb), f32(zeta), f32(energy), qmax, d, 5.0, tau)
        if tau is None:
            assert float(st[0]) == pytest.approx(ref["tau"], rel=1e-5)
            if np.abs(f32(mb) - ref["tau"]).min() < 1e-4 * abs(ref["tau"]):
                continue
        assert np.array_equal(bm.cpu().numpy().astype(bool), ref["unified"])
        assert np.array_equal(tm.cpu().numpy().astype(bool), np.repeat(ref["unified"], 8))
        s = st.cpu().numpy().astype(np.float64)
        assert int(s[5]) == ref["retained"] and int(s[6]) == ref["perfect"] and int(s[7]) == ref["statistical"]
        if tau is not None:
            assert ref["perfect"] + ref["statistical"] == int((kind != 0).sum())
        for i, key in ((1, "zeta_mean"), (3, "zeta_min"), (4, "zeta_max_observed"), (8, "z_max")):
            assert s[i] == pytest.approx(ref[key], rel=1e-5), key
        if nb > 1:
            assert s[2] == pytest.approx(ref["zeta_std"], rel=1e-4)


def _gap_tau(vals):
    v = np.sort(vals.ravel())
    gaps = v[1:] - v[:-1]
    i = int(np.argmax(gaps[len(v) // 4:3 * len(v) // 4])) + len(v) // 4
    return float(0.5 * (v[i] + v[i + 1]))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("sq", [1, 3, 70])
def test_compact_forward_vs_oracle(dtype, sq):
    from orthocache_gpu import orthocache_forward
    nb, H, d = 16, 4, 128
    k = _keys(nb, H, d, {1, 2, 5, 8, 9, 13}, seed=sq, dtype=dtype)
    g = torch.Generator().manual_seed(sq)
    v = torch.randn((nb * 512, H, d), generator=g).to(TD[dtype])
    q = torch.randn((sq, H, d), generator=g).to(TD[dtype])
    probe = O.block_spectra(np64(k), np64(q))
    tau = _gap_tau(probe["max_bound"][probe["zeta"] <= 5.0])  # splits the smooth blocks' bounds
    out, meta = orthocache_forward(q.to(DEV), k.to(DEV), v.to(DEV), zeta_max=5.0, tau=tau, mode="compact")
    ref, info = O.compact_forward(np64(q), np64(k), np64(v), zeta_max=5.0, tau=tau)
    assert out.dtype == torch.bfloat16 and out.shape == (sq, H, d)
    assert_out(out, ref, "bf16", f"compact forward sq={sq}")
    assert 0 < info["retained"] < nb
    assert meta["blocks_retained"] == info["retained"] and meta["compact_num_active"] == info["retained"]
    assert meta["blocks_evicted"] == nb - info["retained"]
    assert meta["eviction_rate"] == pytest.approx(1 - info["retained"] / nb)
    assert meta["tau"] == tau and meta["tau_auto"] is False
    for key in ("zeta_mean", "zeta_std", "zeta_min", "zeta_max_observed"):
        assert meta[key] == pytest.approx(info[key], rel=1e-4), key
    assert meta["perfect_eviction_blocks"] == info["perfect"]
    assert meta["statistical_eviction_blocks"] == info["statistical"]
    for key in ("spectral_ms", "attention_ms", "total_ms", "actual_mode"):
        assert key in meta


def test_compact_auto_tau_bypass_and_zero_active():
    from orthocache_gpu import orthocache_forward
    nb, H, d = 8, 2, 64
    k = _keys(nb, H, d, {3}, seed=9, dtype="f32")
    g = torch.Generator().manual_seed(9)
    v = torch.randn((nb * 512, H, d), generator=g)
    q = torch.randn((2, H, d), generator=g)
    out, meta = orthocache_forward(q.to(DEV), k.to(DEV), v.to(DEV), mode="compact")
    ref, info = O.compact_forward(np64(q), np64(k), np64(v))
    assert meta["tau_auto"] is True and meta["tau"] == pytest.approx(info["tau"], rel=1e-5)
    mb = info["spectra"]["max_bound"]
    if np.abs(mb - info["tau"]).min() > 1e-4 * abs(info["tau"]):
        assert meta["blocks_retained"] == info["retained"]
        assert_out(out, ref, "bf16", "compact forward auto tau")
    # nothing passes the zeta gate: zeros in q's dtype
    out0, meta0 = orthocache_forward(q.to(DEV), k.to(DEV), v.to(DEV), mode="compact", zeta_max=-1.0, tau=-1e30)
    assert meta0["blocks_retained"] == 0 and not out0.any() and out0.dtype == q.dtype
    # under the MI355X crossover (1024 keys): dense attention, bypass flags
    out_b, meta_b = orthocache_forward(q.to(DEV), k[:512].to(DEV), v[:512].to(DEV), mode="compact")
    assert meta_b["bypass_flags"] & 1 and meta_b["eviction_rate"] == 0.0
    dense = np.stack([O.dense_decode(np64(q[:, h]), np.repeat(np64(k[None, :512, h]), 2, 0),
                                     np.repeat(np64(v[None, :512, h]), 2, 0)) for h in range(H)], axis=1)
    np.testing.assert_allclose(np64(out_b), dense, atol=1e-5, rtol=1e-5)


def _walsh_coherent(head_dim, seed, scale=0.5):
    """sum of the natural-order Walsh rows 1..15 of length 512 with N(0, scale^2) coefficients"""
    rng = np.random.RandomState(seed)
    i = np.arange(512)
    blk = np.zeros((512, head_dim))
    for j in range(1, 16):
        w = np.where(np.vectorize(lambda x: bin(x & j).count("1") % 2)(i), -1.0, 1.0)
        blk += np.outer(w, rng.randn(head_dim) * scale)
    return blk


def test_zeta_separates_coherent_from_noise_at_equal_variance():
    """tests/test_spectral_bands.py:130-218 of the reference: a Walsh-coherent
    block has zeta < 0.01, white noise scaled to the same spatial variance has
    zeta > 1 -- no spatial statistic tells them apart."""
    from orthocache_gpu.spectral_energy import compute_spectral_decay_ratio, compute_spectral_bands
    a = _walsh_coherent(64, 2026)
    b = np.random.RandomState(42).randn(512, 64)
    ma, mb = a.mean(0), b.mean(0)
    b = mb + (b - mb) * np.sqrt(np.sum((a - ma) ** 2) / np.sum((b - mb) ** 2))
    k = torch.from_numpy(np.stack([a, b])[:, :, None, :].reshape(1024, 1, 64).astype(np.float32)).to(DEV)
    z = np64(compute_spectral_decay_ratio(k))[:, 0]
    assert z[0] < 0.01 and z[1] > 1.0
    dc, lo, mid, hi = compute_spectral_bands(k)
    total = np64(lo + mid + hi)[:, 0] + np.sum(np64(dc) ** 2, axis=-1)[:, 0]
    np.testing.assert_allclose(total, np.sum(np64(k).reshape(2, 512, 64) ** 2, axis=(1, 2)), rtol=1e-5)


def test_multiband_mask_applies_both_gates():
    """tests/test_spectral_bands.py:220-: block 0 alternating-sign noise is
    evicted by the zeta gate even with a bound gate that passes everything."""
    from orthocache_gpu.spectral_energy import compute_multiband_mask, compute_query_aware_mask
    rng = np.random.RandomState(42)
    keys = rng.randn(1024, 1, 64).astype(np.float32)
    keys[:512, 0, :] *= np.where(np.arange(512) % 2 == 0, 5.0, -5.0)[:, None]
    q = rng.randn(1, 1, 64).astype(np.float32)
    kd, qd = torch.from_numpy(keys).to(DEV), torch.from_numpy(q).to(DEV)
    m = compute_multiband_mask(qd, kd, -100.0, 1.0).cpu().numpy()
    ref = O.block_spectra(keys, q)
    assert np.array_equal(m, (ref["max_bound"] >= -100.0) & (ref["zeta"] <= 1.0))
    assert not m[0, 0]
    assert compute_query_aware_mask(qd, kd, -100.0).all()


def test_orthocache_attention_api():
    """tests/test_adaptive_attention.py of the reference: stream compaction of
    all-active / all-evicted masks, zeros (q's dtype) when nothing is active,
    bfloat16 (seq_q, heads, d) output, the eviction-rate statistic, and every
    block active equal to dense attention."""
    from orthocache_gpu.adaptive_attention import orthocache_attention, stream_compact
    idx, n = stream_compact(torch.ones(6, dtype=torch.bool, device=DEV))
    assert n == 6 and idx.tolist() == list(range(6))
    idx, n = stream_compact(torch.zeros(6, dtype=torch.bool, device=DEV))
    assert n == 0 and idx.tolist() == list(range(6))
    idx, n = stream_compact(torch.tensor([False, True, False, True], device=DEV))
    assert n == 2 and idx.tolist() == [1, 3, 0, 2]
    g = torch.Generator().manual_seed(5)
    q = torch.randn((3, 2, 64), generator=g).to(DEV)
    k = torch.randn((2048, 2, 64), generator=g).to(DEV)
    v = torch.randn((2048, 2, 64), generator=g).to(DEV)
    out, st = orthocache_attention(q, k, v, torch.zeros(4, dtype=torch.bool, device=DEV))
    assert not out.any() and out.dtype == q.dtype and st["num_active"] == 0 and st["eviction_rate"] == 1.0
    out, st = orthocache_attention(q, k, v, torch.tensor([True, False, True, True], device=DEV))
    assert out.dtype == torch.bfloat16 and out.shape == (3, 2, 64)
    assert st["num_active"] == 3 and st["num_blocks"] == 4 and st["eviction_rate"] == pytest.approx(0.25)
    out, _ = orthocache_attention(q, k, v, torch.ones(4, dtype=torch.bool, device=DEV))
    dense = np.stack([O.dense_decode(np64(q[:, h]), np.repeat(np64(k[None, :, h]), 3, 0),
                                     np.repeat(np64(v[None, :, h]), 3, 0)) for h in range(2)], axis=1)
    assert_out(out, dense, "bf16", "orthocache_attention all blocks")


def test_orthocache_attention_batched():
    from orthocache_gpu.adaptive_attention import orthocache_attention, orthocache_attention_batched
    g = torch.Generator().manual_seed(6)
    q = torch.randn((2, 3, 2, 64), generator=g).to(DEV)
    k = torch.randn((2, 1536, 2, 64), generator=g).to(DEV)
    v = torch.randn((2, 1536, 2, 64), generator=g).to(DEV)
    mask = torch.tensor([True, False, True], device=DEV)
    out, st = orthocache_attention_batched(q, k, v, mask)
    assert out.shape == (2, 3, 2, 64) and out.dtype == torch.bfloat16
    assert st["batch_size"] == 2 and st["num_active"] == 2 and st["eviction_rate"] == pytest.approx(1 / 3)
    for b in range(2):
        one, _ = orthocache_attention(q[b], k[b], v[b], mask)
        assert torch.equal(out[b], one)
    zero, st0 = orthocache_attention_batched(q, k, v, torch.zeros(3, dtype=torch.bool, device=DEV))
    assert not zero.any() and st0["num_active"] == 0
