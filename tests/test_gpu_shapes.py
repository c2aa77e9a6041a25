"""GPU parity of the portable kernels (oc_generic.hip): head dims other than
64 / 128 and tiles other than 64 tokens, which the reference accepts as
powers of two (fused_eviction.py:609-610, gqa_eviction.py:551-552,
paged_eviction.py:345-347).

* The reference-written golden cases at such shapes (tests/golden/shapes_*)
  through the drop-in entry points: masks and counts equal, outputs within
  the north-star bar.
* Random cases against the oracle over head_dim {16, 32, 256, 512} x tile
  {16, 32, 64, 128, 256} x gate {zeta, cs} x mode {single pass, cached} x
  dtype, with G up to 12 (two head chunks), fp8 K/V with per-tile scales,
  bf16 V beside fp8 K, OC_KSCALE_DEQUANT, row lengths with partial tails,
  the mask gate and the per-split partials.
* oc_decode's `portable` switch on the tuned kernels' own shapes (head_dim
  128, 64-token tiles): the same masks and, within the bar, the same outputs
  as the tuned kernels on the same inputs.
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
    if dt == "f32":
        return torch.from_numpy(raw.astype(np.float32)).to(DEV)
    if dt in ("f16", "bf16"):
        return torch.from_numpy(raw.astype(np.uint16).view(np.int16)).view(TORCH_DT[dt]).to(DEV)
    if dt == "i32":
        return torch.from_numpy(raw.astype(np.int32)).to(DEV)
    raise ValueError(dt)


def mixed(rows, n_tiles, d, ts, seed, noise_frac=0.5):
    """(rows, n_tiles * ts, d) float32 keys: smooth tiles W_ts C (rows 1..4
    of C) plus 0.05 N(0, 1), noise tiles W_ts C with rows [min(32, ts/2), ts)
    of C, in random order per row; returns (keys, noise labels)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.from_numpy(O.walsh_matrix(ts))
    hi0, lo_end = min(32, ts // 2), min(5, ts)
    keys = torch.empty(rows, n_tiles * ts, d)
    noise = torch.zeros(rows, n_tiles, dtype=torch.bool)
    for r in range(rows):
        lab = torch.randperm(n_tiles, generator=g) < int(round(noise_frac * n_tiles))
        for t in range(n_tiles):
            c = torch.zeros(ts, d)
            if lab[t]:
                c[hi0:] = torch.randn(ts - hi0, d, generator=g)
                tile = w @ c
            else:
                c[1:lo_end] = torch.randn(lo_end - 1, d, generator=g)
                tile = w @ c + 0.05 * torch.randn(ts, d, generator=g)
            keys[r, t * ts:(t + 1) * ts] = tile
        noise[r] = lab
    return keys, noise


def round_np(x, dt):
    return np32(torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(TORCH_DT[dt]))


# ---------------------------------------------------------------- golden cases

@pytest.mark.parametrize("ts", [16, 32, 128, 256])
def test_golden_scores_shapes(ts):
    from orthocache_gpu import triton_fwht_eviction
    raw, dec, dt, meta, params, _ = golden_io.load(f"shapes_fwht_ts{ts}")
    mask, zeta = triton_fwht_eviction(to_dev(raw["keys"], dt["keys"]), params["zeta_max"], tile_size=ts,
                                      return_zeta=True)
    assert np.array_equal(mask.cpu().numpy(), dec["mask"].astype(bool))
    np.testing.assert_allclose(zeta.cpu().numpy(), dec["zeta"], rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("name", ["shapes_v1_d32", "shapes_v1_ts128"])
def test_golden_v1_shapes(name):
    from orthocache_gpu import fused_orthocache_attention
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention(to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]),
                                        to_dev(raw["values"], dt["values"]), params["zeta_max"],
                                        tile_size=params["tile_size"], return_mask=True)
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), meta["eviction_mask"])
    for k in ("tiles_retained", "tiles_evicted", "eviction_rate"):
        assert m[k] == meta[k]
    assert_out(out, dec["out"], dt["out"], name, ref_rounded=True)


@pytest.mark.parametrize("name", ["shapes_v2_d256_bf16", "shapes_v2_d32_f16", "shapes_v2_d16_ts16_f32",
                                  "shapes_v2_ts32_f32", "shapes_v2_ts128_bf16"])
def test_golden_v2_shapes(name):
    from orthocache_gpu import fused_orthocache_attention_v2
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_v2(to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]),
                                           to_dev(raw["values"], dt["values"]), params["zeta_max"],
                                           tile_size=params["tile_size"])
    for k, v in meta.items():
        assert m[k] == v, k
    assert_out(out, dec["out"], dt["out"], name, ref_rounded=True)


@pytest.mark.parametrize("name", ["shapes_v3_d256_f32", "shapes_v3_ts128_bf16", "shapes_v3_ts32_f32"])
def test_golden_v3_shapes(name):
    from orthocache_gpu import fused_orthocache_attention_v3_gqa
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_v3_gqa(
        to_dev(raw["q"], dt["q"]), to_dev(raw["keys"], dt["keys"]), to_dev(raw["values"], dt["values"]),
        params["tau"], params["G"], tile_size=params["tile_size"])
    for k, v in meta.items():
        assert m[k] == v, k
    assert_out(out, dec["out"], dt["out"], name, ref_rounded=True)


@pytest.mark.parametrize("name", ["shapes_paged_d256", "shapes_paged_ts128", "shapes_paged_d32_ts32"])
def test_golden_paged_shapes(name):
    from orthocache_gpu import fused_orthocache_attention_paged
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = fused_orthocache_attention_paged(
        to_dev(raw["q"], dt["q"]), to_dev(raw["k_cache"], dt["k_cache"]), to_dev(raw["v_cache"], dt["v_cache"]),
        to_dev(raw["block_tables"], "i32"), params["zeta_max"], tile_size=params["tile_size"])
    assert_out(out, dec["out"], dt["out"], name, ref_rounded=True)


# ---------------------------------------------------------------- random cases vs the oracle

SHAPES = [(16, 64), (32, 64), (256, 64), (512, 32), (128, 16), (64, 32), (128, 128), (32, 256)]


@pytest.mark.parametrize("d,ts", SHAPES, ids=lambda x: str(x))
@pytest.mark.parametrize("mode", ["single_pass", "cached"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_v2_zeta_shapes_vs_oracle(d, ts, mode, dtype):
    """v2 (zeta gate, one head per row), 3 heads x 7 tiles, explicit splits
    (2 and the default): mask bit-exact, output within the bar."""
    from orthocache_gpu import fused_orthocache_attention_v2, score_tiles
    k, noise = mixed(3, 7, d, ts, seed=d + ts)
    v = torch.randn(3, 7 * ts, d, generator=torch.Generator().manual_seed(d * ts))
    q = torch.randn(3, d, generator=torch.Generator().manual_seed(d + 3 * ts))
    kd, vd, qd = (x.to(TORCH_DT[dtype]).to(DEV) for x in (k, v, q))
    ref, rmeta, rmask = O.fused_v2(np32(qd), np32(kd), np32(vd), 5.0, tile_size=ts)
    sc = score_tiles(kd, tile_size=ts) if mode == "cached" else None
    print(f"v2 shapes d={d} ts={ts} {mode} {dtype}", flush=True)
    for P in (None, 2):
        out, m = fused_orthocache_attention_v2(qd, kd, vd, 5.0, num_splits=P, tile_size=ts, mode=mode,
                                               score_cache=sc)
        assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask), (P, mode)
        assert m["tiles_evicted"] == rmeta["tiles_evicted"]
        assert_out(out, ref, dtype, f"portable v2 d={d} ts={ts} {mode} {dtype} P={P}")
    if ts > 32:
        assert np.array_equal(rmask, ~noise.numpy())


@pytest.mark.parametrize("d,ts", [(32, 64), (256, 64), (64, 128), (512, 64), (128, 256)], ids=lambda x: str(x))
@pytest.mark.parametrize("G", [1, 4, 12])
@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_v3_cs_shapes_vs_oracle(d, ts, G, mode):
    """v3 (Cauchy-Schwarz gate), 2 kv heads, G query heads (12: two head
    chunks of the portable kernel), bf16, tau between the tile clusters."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    k, noise = mixed(2, 6, d, ts, seed=7 * d + ts)
    g = torch.Generator().manual_seed(G * d + ts)
    v = torch.randn(2, 6 * ts, d, generator=g)
    q = torch.randn(2 * G, d, generator=g)
    kd, vd, qd = (x.to(torch.bfloat16).to(DEV) for x in (k, v, q))
    # tau midway between the largest smooth and the smallest noise bound
    _, _, _, eh = O.fwht_scores(np32(kd).reshape(-1, d), 0.0, tile_size=ts)
    eh = eh.reshape(2, 6)
    qn = np.array([O.q_norms(np32(qd)[h * G:(h + 1) * G]).max() for h in range(2)])
    b = qn[:, None] * np.sqrt(eh)
    tau = float(0.5 * (b[~noise.numpy()].max() + b[noise.numpy()].min()))
    ref, rmeta, rmask = O.gqa_v3(np32(qd), np32(kd), np32(vd), tau, G, tile_size=ts)
    assert np.array_equal(rmask, noise.numpy())  # the gate keeps the tiles with high-band energy
    sc = score_tiles(kd, tile_size=ts) if mode == "cached" else None
    print(f"v3 shapes d={d} ts={ts} G={G} {mode}", flush=True)
    out, m = fused_orthocache_attention_v3_gqa(qd, kd, vd, tau, G, tile_size=ts, mode=mode, score_cache=sc)
    assert np.array_equal(m["eviction_mask"].cpu().numpy(), rmask)
    assert_out(out, ref, "bf16", f"portable v3 d={d} ts={ts} G={G} {mode}")


@pytest.mark.parametrize("d,ts,bs", [(256, 64, 16), (32, 128, 32), (64, 32, 8)], ids=lambda x: str(x))
@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_paged_shapes_lengths_vs_oracle(d, ts, bs, mode):
    """Paged GQA at other shapes: 3 sequences x 2 kv heads, G = 4, lengths
    with partial tail tiles, shuffled pool; the Cauchy-Schwarz gate at a
    calibrated tau, against the oracle's generalised decode."""
    from orthocache_gpu import fused_orthocache_attention_paged, score_paged_tiles
    from orthocache_gpu.workloads import paged_pool
    B, hkv, G, T = 3, 2, 4, 5
    k, noise = mixed(B * hkv, T, d, ts, seed=3 * d + ts + bs)
    g = torch.Generator().manual_seed(d + ts + bs)
    v = torch.randn(B * hkv, T * ts, d, generator=g)
    q = torch.randn(B * hkv * G, d, generator=g)
    lens = [T * ts, 2 * ts + ts // 2 + 1, ts + 3]
    kc, vc, bt = paged_pool(k, v, hkv, bs, lens, seed=d + bs)
    row_lens = [lens[r // hkv] for r in range(B * hkv)]
    _, _, _, eh = O.fwht_scores(k.numpy().reshape(-1, d), 0.0, tile_size=ts)
    eh = eh.reshape(B * hkv, T)
    qn = np.array([O.q_norms(q.numpy()[r * G:(r + 1) * G]).max() for r in range(B * hkv)])
    bnd = qn[:, None] * np.sqrt(eh)
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    ref = O.decode_rows(q.numpy(), k.numpy(), v.numpy(), gate="cs", threshold=tau, G=G, tile_size=ts,
                        lengths=row_lens)
    lt = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sc = score_paged_tiles(kc.to(DEV), bt.to(DEV), tile_size=ts, context_lens=lt) if mode == "cached" else None
    print(f"paged shapes d={d} ts={ts} bs={bs} {mode}", flush=True)
    out, m = fused_orthocache_attention_paged(q.view(B, hkv * G, d).to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                              5.0, tile_size=ts, num_query_groups=G, tau=tau, context_lens=lt,
                                              mode=mode, score_cache=sc)
    assert m["tiles_retained"] == ref["retained"] and m["tiles_evicted"] == ref["evicted"]
    assert_out(out.view(B * hkv * G, d), ref["out"], "f32", f"portable paged d={d} ts={ts} bs={bs} {mode}")


@pytest.mark.parametrize("d,ts", [(256, 64), (32, 128)], ids=lambda x: str(x))
def test_fp8_tile_scales_and_bf16_v_shapes(d, ts):
    """fp8-e4m3 K and V with one scale per (row, tile), scoring and logits
    on the dequantised values; and a paged fp8 K beside a bf16 V with a
    scalar k_scale (in-kernel dequantisation, V read as bf16)."""
    from orthocache_gpu import fused_orthocache_attention_v3_gqa, score_tiles
    from orthocache_gpu.workloads import quantize_fp8_tiles
    G = 4
    k, noise = mixed(2, 6, d, ts, seed=11 * d + ts)
    g = torch.Generator().manual_seed(5 * d + ts)
    v = torch.randn(2, 6 * ts, d, generator=g)
    q = torch.randn(2 * G, d, generator=g).to(torch.bfloat16)

    def tile_quant(x):  # per (row, ts-token tile): amax / 448
        t = x.view(x.shape[0], -1, ts, d)
        amax = t.abs().amax(dim=(2, 3))
        s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
        return (t / s[..., None, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(x.shape), s.float()
    kq, ks = tile_quant(k)
    vq, vs = tile_quant(v)
    tab = O.fp8_e4m3fn_table()
    kf, vf = tab[kq.view(torch.uint8).numpy()], tab[vq.view(torch.uint8).numpy()]
    probe = O.decode_rows(np32(q), kf, vf, gate="cs", threshold=-1.0, G=G, tile_size=ts, k_scales=ks.numpy(),
                          v_scales=vs.numpy())
    kdeq = (torch.from_numpy(kf).view(2, 6, ts, d) * ks[..., None, None]).numpy().reshape(-1, d)
    _, _, _, eh = O.fwht_scores(kdeq, 0.0, tile_size=ts)
    qn = np.array([O.q_norms(np32(q)[h * G:(h + 1) * G]).max() for h in range(2)])
    bnd = qn[:, None] * np.sqrt(eh.reshape(2, 6))
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    ref = O.decode_rows(np32(q), kf, vf, gate="cs", threshold=tau, G=G, tile_size=ts, k_scales=ks.numpy(),
                        v_scales=vs.numpy())
    assert probe["keep"].all() and np.array_equal(ref["keep"], noise.numpy())
    kd, vd, ksd, vsd = kq.to(DEV), vq.to(DEV), ks.to(DEV), vs.to(DEV)
    sc = score_tiles(kd, k_scale=ksd, tile_size=ts)
    for mode in ("single_pass", "cached"):
        out, m = fused_orthocache_attention_v3_gqa(q.to(DEV), kd, vd, tau, G, k_scale=ksd, v_scale=vsd,
                                                   tile_size=ts, mode=mode, score_cache=sc)
        assert np.array_equal(m["eviction_mask"].cpu().numpy(), ref["keep"]), mode
        assert_out(out, ref["out"], "fp8", f"portable fp8 d={d} ts={ts} {mode}")
    # paged fp8 K beside a bf16 V with a scalar k_scale (the reference's
    # paged fp8 cache, paged_eviction.py:354-357): bf16 q, cached mode, K
    # dequantised in the kernel as bf16(float(fp8) * k_scale), V read as bf16
    from orthocache_gpu import fused_orthocache_attention_paged
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    from orthocache_gpu.workloads import paged_pool
    kc, vc, bt = paged_pool(k, v.to(torch.bfloat16), 2, 16, [6 * ts], seed=ts)
    amax = kc.abs().max().item()
    ksc = amax / 448.0
    kc8 = (kc / ksc).clamp(-448, 448).to(torch.float8_e4m3fn)
    qp = q[:2].reshape(1, 2, d)  # the reference's paged path: one query head per kv head
    ref3, _, mask3 = O.paged(np32(qp), tab[kc8.view(torch.uint8).numpy()], np32(vc), bt.numpy(), 5.0,
                             tile_size=ts, k_scale=ksc, q_dtype="bf16", k_is_fp8=True)
    sc3 = score_paged_tiles(kc8.to(DEV), bt.to(DEV), tile_size=ts, k_scale=ksc, q_dtype=torch.bfloat16)
    out, m = fused_orthocache_attention_paged(qp.to(DEV), kc8.to(DEV), vc.to(DEV), bt.to(DEV), 5.0, k_scale=ksc,
                                              tile_size=ts, mode="cached", score_cache=sc3)
    assert m["tiles_retained"] == int(mask3.sum())
    assert_out(out, ref3, "fp8", f"portable paged fp8 K + bf16 V d={d} ts={ts}")


@pytest.mark.parametrize("d,ts", [(256, 64), (32, 32)], ids=lambda x: str(x))
def test_partials_and_mask_gate_shapes(d, ts):
    """return_partials (one partial per logical split) against the oracle's
    per-split states, and the mask gate (block-sparse path) at other shapes."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    k, _ = mixed(2, 9, d, ts, seed=d + 2 * ts)
    g = torch.Generator().manual_seed(d + 5 * ts)
    v = torch.randn(2, 9 * ts, d, generator=g)
    q = torch.randn(2, d, generator=g)
    kv = X.rows_layout(k.to(DEV), v.to(DEV), tile_size=ts)
    res = X.decode(kv, q.to(DEV), 1, gate=N.OC_GATE_ZETA, threshold=5.0, num_splits=4, out_dtype=torch.float32,
                   want_partials=True)
    torch.cuda.synchronize()
    ref = O.decode_rows(q.numpy(), k.numpy(), v.numpy(), gate="zeta", threshold=5.0, G=1, tile_size=ts,
                        num_splits=4, want_partials=True)
    pm, pl, pacc = (np32(t) for t in res.partials)
    # the partial states: float32 sums in another order, so relative bars
    assert np.array_equal(pm == np.float32(-1e9), ref["M"] == np.float32(-1e9))  # same empty splits
    np.testing.assert_allclose(pm, ref["M"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pl, ref["L"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(pacc, ref["ACC"], rtol=1e-5, atol=1e-5)
    assert_out(res.out, ref["out"], "f32", f"portable merged d={d} ts={ts}")
    mask = torch.zeros(2, 9, dtype=torch.uint8)
    mask[0, [0, 4, 8]] = 1
    mask[1, [2, 3]] = 1
    res = X.decode(kv, q.to(DEV), 1, gate=N.OC_GATE_MASK, threshold=0.0, mode=N.OC_MODE_CACHED,
                   out_dtype=torch.float32, tile_mask=mask.to(DEV), want_keep=True)
    torch.cuda.synchronize()
    keep = mask.bool().numpy()
    dense = np.stack([O.dense_decode(q.numpy()[r:r + 1], k.numpy()[r:r + 1, np.repeat(keep[r], ts)],
                                     v.numpy()[r:r + 1, np.repeat(keep[r], ts)])[0] for r in range(2)])
    assert np.array_equal(res.keep.cpu().numpy().astype(bool), keep)
    assert_out(res.out, dense, "f32", f"portable mask gate d={d} ts={ts}")


@pytest.mark.parametrize("gate", ["zeta", "cs"])
@pytest.mark.parametrize("mode", ["single_pass", "cached"])
def test_portable_switch_matches_tuned_kernels(gate, mode):
    """oc_decode with portable = 1 on the tuned kernels' own shape (head_dim
    128, 64-token tiles, bf16, G = 4): the same eviction masks as the tuned
    kernels and outputs within the bf16 bar of theirs, on the same inputs."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.triton_kernels.fwht_fused_prototype import score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q
    G = 4 if gate == "cs" else 1
    wl = make_kv(6, 40 * 64, 128, dtype=torch.bfloat16, device=DEV, seed=13)
    q = make_q(6, G, 128, dtype=torch.bfloat16, device=DEV, seed=14)
    sc = score_tiles(wl.keys)
    thr = calibrate_tau(sc.e_high, q, G) if gate == "cs" else 5.0
    gcode = N.OC_GATE_CS if gate == "cs" else N.OC_GATE_ZETA
    mcode = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    kv = X.rows_layout(wl.keys, wl.values)
    outs, keeps = [], []
    for portable in (0, 1):
        res = X.decode(kv, q, G, gate=gcode, threshold=thr, mode=mcode, scores=sc.as_pair(),
                       out_dtype=torch.float32, want_keep=True, portable=portable)
        torch.cuda.synchronize()
        outs.append(res.out)
        keeps.append(res.keep)
    assert torch.equal(keeps[0], keeps[1])
    assert torch.equal(keeps[0][:, :40].bool(), wl.noise if gate == "cs" else ~wl.noise)
    assert_out(outs[1], np32(outs[0]), "f32", f"portable vs tuned {gate} {mode}")


# ------------------------------------------------ head_dim 256, tuned kernel

def _d256_case(rows, T, G, dt, seed):
    k, noise = mixed(rows, T, 256, 64, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    v = torch.randn(rows, T * 64, 256, generator=g)
    q = torch.randn(rows * G, 256, generator=g)
    kd, vd, qd = (x.to(TORCH_DT[dt]).to(DEV) for x in (k, v, q))
    return kd, vd, qd, noise


def _cs_tau(qd, kd, noise, G):
    rows = kd.shape[0]
    _, _, _, eh = O.fwht_scores(np32(kd).reshape(-1, 256), 0.0)
    eh = eh.reshape(rows, -1)
    qn = np.array([O.q_norms(np32(qd)[r * G:(r + 1) * G]).max() for r in range(rows)])
    b = qn[:, None] * np.sqrt(eh)
    return float(0.5 * (b[~noise.numpy()].max() + b[noise.numpy()].min()))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 6, 8, 12])
@pytest.mark.parametrize("gate", ["cs", "zeta", "mask", "none", "cs_single_pass", "zeta_single_pass"])
def test_head_dim_256_tuned_kernel(dt, G, gate):
    """head_dim 256, 64-token tiles, 16-bit K/V with q of K's type, on the
    matrix-core kernels (4-wave workgroups, one wave per SIMD): the cached
    score- or mask-gated decode and the dense decode on the per-wave-prologue
    kernel (a workgroup takes several splits: splits_per_group = 2; G = 6, 8
    merged in two passes of 4 heads), the single-pass gates on the general
    one, and G = 12 on the general one in two chunks of up to 8 heads;
    against the oracle, and against the same decode forced onto the portable
    kernels."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T = 3, 12
    kd, vd, qd, noise = _d256_case(rows, T, G, dt, seed=17 * G + 3 * len(gate))
    kv = X.rows_layout(kd, vd)
    q32, k32, v32 = np32(qd), np32(kd), np32(vd)
    tmask = None
    single = gate.endswith("_single_pass")
    gate = gate.replace("_single_pass", "")
    if gate == "cs":
        thr, ng = _cs_tau(qd, kd, noise, G), N.OC_GATE_CS
    elif gate == "zeta":
        thr, ng = 5.0, N.OC_GATE_ZETA
    elif gate == "mask":
        thr, ng = 0.0, N.OC_GATE_MASK
        tmask = (torch.rand(rows, T, generator=torch.Generator().manual_seed(G)) < 0.5).to(torch.uint8)
        tmask[:, 0] = 1
    else:
        thr, ng = 0.0, N.OC_GATE_NONE
    if gate == "mask":
        keep = tmask.bool().numpy()
        ref = np.zeros((rows * G, 256), dtype=np.float32)
        for r in range(rows):
            sel = np.repeat(keep[r], 64)
            for h in range(G):
                ref[r * G + h] = O.dense_decode(q32[r * G + h:r * G + h + 1], k32[r:r + 1, sel], v32[r:r + 1, sel])[0]
    else:
        res = O.decode_rows(q32, k32, v32, gate="none" if gate == "none" else gate, threshold=thr, G=G)
        ref, keep = res["out"], res["keep"]
        if gate != "none":
            assert np.array_equal(keep, noise.numpy() if gate == "cs" else ~noise.numpy())
    e_low, e_high, _, _ = X.score_tiles(kv)
    mode = N.OC_MODE_SINGLE_PASS if (gate == "none" or single) else N.OC_MODE_CACHED
    outs = {}
    for portable in (0, 1):
        print(f"head_dim 256 {dt} G={G} gate={gate} single={single} portable={portable}", flush=True)
        r = X.decode(kv, qd, G, gate=ng, threshold=thr, mode=mode, scores=(e_low, e_high), num_splits=4,
                     splits_per_group=2, out_dtype=TORCH_DT[dt], want_keep=gate != "none",
                     tile_mask=None if tmask is None else tmask.to(DEV), portable=portable)
        torch.cuda.synchronize()
        if gate != "none":
            assert np.array_equal(r.keep.cpu().numpy().astype(bool), keep), portable
        assert_out(r.out, ref, dt, f"head_dim 256 {'portable' if portable else 'tuned'} {dt} G={G} {gate}"
                                   f"{' single pass' if single else ''}")
        outs[portable] = np32(r.out)
    # the two kernels agree to the output type's rounding
    assert np.max(np.abs(outs[0] - outs[1])) <= {"bf16": 1.6e-2, "f16": 2e-3}[dt]


@pytest.mark.parametrize("G", [4, 8])
def test_head_dim_256_routing_and_full_row(G):
    """With the automatic split grouping, head_dim 256 bf16 cached and dense
    decodes take several splits per workgroup (the tuned kernel's grouping:
    fewer partials than splits) while the same call forced portable keeps one
    split per workgroup; the tuned kernel's output on 8 rows x 10240 tokens
    (160 tiles, P = 40) matches the oracle, both modes, and with one split
    per tile and per workgroup (160 partials per row in the fused merge,
    two passes of 4 heads at G = 8)."""
    import ctypes
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T = 8, 160
    kd, vd, qd, noise = _d256_case(rows, T, G, "bf16", seed=2560 + G)
    kv = X.rows_layout(kd, vd)
    tau = _cs_tau(qd, kd, noise, G)
    e_low, e_high, _, _ = X.score_tiles(kv)
    P = X.auto_num_splits(T, qd.device)
    lib = N.lib()
    groups = {}
    for portable in (0, 1):
        p = N.OcDecodeParams()
        p.kv = kv.struct()
        p.q, p.q_dtype, p.G, p.q_row_stride = qd.data_ptr(), N.OC_BF16, G, qd.stride(0)
        p.gate, p.mode, p.threshold = N.OC_GATE_CS, N.OC_MODE_CACHED, tau
        p.score_e_low, p.score_e_high, p.score_row_stride = e_low.data_ptr(), e_high.data_ptr(), e_high.stride(0)
        p.num_splits, p.out_dtype, p.portable = P, N.OC_BF16, portable
        groups[portable] = lib.oc_decode_num_groups(ctypes.byref(p))
    assert groups[1] == P and groups[0] < P, (P, groups)
    q32, k32, v32 = np32(qd), np32(kd), np32(vd)
    for gate, ng, mode, ns, spg in (("cs", N.OC_GATE_CS, N.OC_MODE_CACHED, P, 0),
                                    ("none", N.OC_GATE_NONE, N.OC_MODE_SINGLE_PASS, P, 0),
                                    ("cs", N.OC_GATE_CS, N.OC_MODE_CACHED, T, 1)):
        ref = O.decode_rows(q32, k32, v32, gate=gate, threshold=tau, G=G)
        print(f"head_dim 256 full row G={G} {gate} P={ns} spg={spg}", flush=True)
        r = X.decode(kv, qd, G, gate=ng, threshold=tau, mode=mode, scores=(e_low, e_high), num_splits=ns,
                     splits_per_group=spg, out_dtype=torch.bfloat16, want_keep=gate == "cs")
        torch.cuda.synchronize()
        if gate == "cs":
            assert np.array_equal(r.keep.cpu().numpy().astype(bool), ref["keep"])
        assert_out(r.out, ref["out"], "bf16", f"head_dim 256 tuned full row G={G} {gate} P={ns} spg={spg}")


@pytest.mark.parametrize("G", [4, 8])
def test_head_dim_256_partials_single_pass(G):
    """return_partials at head_dim 256 (one workgroup per logical split, the
    general matrix-core kernel, single-pass CS gate; 8 heads in one
    workgroup): every split's (m, l, acc) against the oracle's, and the
    merged output."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T = 2, 9
    kd, vd, qd, noise = _d256_case(rows, T, G, "bf16", seed=99 + G)
    kv = X.rows_layout(kd, vd)
    tau = _cs_tau(qd, kd, noise, G)
    print(f"head_dim 256 partials G={G}", flush=True)
    res = X.decode(kv, qd, G, gate=N.OC_GATE_CS, threshold=tau, num_splits=4, out_dtype=torch.float32,
                   want_partials=True, want_keep=True)
    torch.cuda.synchronize()
    ref = O.decode_rows(np32(qd), np32(kd), np32(vd), gate="cs", threshold=tau, G=G, num_splits=4,
                        want_partials=True)
    assert np.array_equal(res.keep.cpu().numpy().astype(bool), ref["keep"])
    pm, pl, pacc = (np32(t) for t in res.partials)
    assert np.array_equal(pm == np.float32(-1e9), ref["M"] == np.float32(-1e9))
    np.testing.assert_allclose(pm, ref["M"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pl, ref["L"], rtol=1e-5, atol=1e-6)
    # the matrix-core p.V keeps about 16 bits of each p (a 16-bit high part
    # plus the 16-bit rounding of the rest): errors of 2^-17 of |p v| per
    # product, so the accumulator bar scales with the partials' magnitude
    scale = float(np.abs(ref["ACC"]).max())
    np.testing.assert_allclose(pacc, ref["ACC"], rtol=1e-5, atol=1e-5 * max(1.0, scale))
    assert_out(res.out, ref["out"], "f32", "head_dim 256 tuned partials merged")


@pytest.mark.parametrize("bs", [16, 64])
@pytest.mark.parametrize("mode", ["cached", "single_pass", "dense"])
def test_head_dim_256_paged_tuned(bs, mode):
    """head_dim 256 paged bf16 decode on the matrix-core kernels: 3 sequences
    x 2 kv heads, G = 4, row lengths with partial tail tiles (the flat layout
    of rows of different lengths for the cached and dense decodes), a
    shuffled pool with 16- and 64-token pages; the Cauchy-Schwarz gate at a
    calibrated tau, against the oracle's decode over the rows' lengths."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import paged_pool
    B, hkv, G, T, d = 3, 2, 4, 14, 256
    k, noise = mixed(B * hkv, T, d, 64, seed=256 + bs)
    g = torch.Generator().manual_seed(bs)
    v = torch.randn(B * hkv, T * 64, d, generator=g)
    q = torch.randn(B * hkv * G, d, generator=g)
    k, v, q = (x.to(torch.bfloat16) for x in (k, v, q))
    lens = [T * 64, 9 * 64 + 37, 3 * 64 + 5]
    kc, vc, bt = paged_pool(k, v, hkv, bs, lens, seed=bs)
    row_lens = [lens[r // hkv] for r in range(B * hkv)]
    k32, v32, q32 = np32(k), np32(v), np32(q)
    _, _, _, eh = O.fwht_scores(k32.reshape(-1, d), 0.0)
    eh = eh.reshape(B * hkv, T)
    qn = np.array([O.q_norms(q32[r * G:(r + 1) * G]).max() for r in range(B * hkv)])
    bnd = qn[:, None] * np.sqrt(eh)
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    gate = "none" if mode == "dense" else "cs"
    ref = O.decode_rows(q32, k32, v32, gate=gate, threshold=tau, G=G, lengths=row_lens)
    kv = X.paged_layout(kc.to(DEV), vc.to(DEV), bt.to(DEV), T)
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    e_low, e_high, _, _ = X.score_tiles(kv)
    ng = N.OC_GATE_NONE if mode == "dense" else N.OC_GATE_CS
    nm = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    print(f"head_dim 256 paged bs={bs} {mode}", flush=True)
    r = X.decode(kv, q.to(DEV), G, gate=ng, threshold=tau, mode=nm, scores=(e_low, e_high),
                 out_dtype=torch.float32, want_keep=mode != "dense")
    torch.cuda.synchronize()
    if mode != "dense":
        keep = r.keep.cpu().numpy().astype(bool)
        for row in range(B * hkv):
            nt = -(-row_lens[row] // 64)
            assert np.array_equal(keep[row, :nt], ref["keep"][row, :nt]), row
    assert_out(r.out, ref["out"], "f32", f"head_dim 256 tuned paged bs={bs} {mode}")


def _tile_quant(x, ts=64):
    """per (row, ts-token tile) fp8-e4m3 with scale amax / 448"""
    d = x.shape[-1]
    t = x.view(x.shape[0], -1, ts, d)
    amax = t.abs().amax(dim=(2, 3))
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    return (t / s[..., None, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(x.shape), s.float()


@pytest.mark.parametrize("G", [1, 4, 8])
@pytest.mark.parametrize("mode", ["cached", "single_pass", "dense"])
def test_head_dim_256_fp8_tile_scales_tuned(G, mode):
    """head_dim 256 fp8-e4m3 K and V with one scale per (row, tile) and bf16
    q on the matrix-core kernels (K widened per instruction, V through the
    transposing 8-bit LDS read): masks and outputs against the oracle on the
    decoded values times their scales."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T, d = 3, 12, 256
    k, noise = mixed(rows, T, d, 64, seed=80 + G)
    g = torch.Generator().manual_seed(81 + G)
    v = torch.randn(rows, T * 64, d, generator=g)
    q = torch.randn(rows * G, d, generator=g).to(torch.bfloat16)
    kq, ks = _tile_quant(k)
    vq, vs = _tile_quant(v)
    tab = O.fp8_e4m3fn_table()
    kf, vf = tab[kq.view(torch.uint8).numpy()], tab[vq.view(torch.uint8).numpy()]
    kdeq = (torch.from_numpy(kf).view(rows, T, 64, d) * ks[..., None, None]).numpy().reshape(-1, d)
    _, _, _, eh = O.fwht_scores(kdeq, 0.0)
    qn = np.array([O.q_norms(np32(q)[r * G:(r + 1) * G]).max() for r in range(rows)])
    bnd = qn[:, None] * np.sqrt(eh.reshape(rows, T))
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    gate = "none" if mode == "dense" else "cs"
    ref = O.decode_rows(np32(q), kf, vf, gate=gate, threshold=tau, G=G, k_scales=ks.numpy(), v_scales=vs.numpy())
    kv = X.rows_layout(kq.to(DEV), vq.to(DEV))
    kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(ks.to(DEV), rows, T, DEV)
    kv.v_scale_mode, kv.v_scales = X.vscale_mode(vs.to(DEV), rows, T, DEV)
    e_low, e_high, _, _ = X.score_tiles(kv)
    ng = N.OC_GATE_NONE if mode == "dense" else N.OC_GATE_CS
    nm = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    print(f"head_dim 256 fp8 tile scales G={G} {mode}", flush=True)
    r = X.decode(kv, q.to(DEV), G, gate=ng, threshold=tau, mode=nm, scores=(e_low, e_high), num_splits=4,
                 splits_per_group=2, out_dtype=torch.float32, want_keep=mode != "dense")
    torch.cuda.synchronize()
    if mode != "dense":
        assert np.array_equal(r.keep.cpu().numpy().astype(bool), ref["keep"])
        assert np.array_equal(ref["keep"], noise.numpy())
    assert_out(r.out, ref["out"], "fp8", f"head_dim 256 tuned fp8 tile scales G={G} {mode}")


@pytest.mark.parametrize("G", [4, 8])
@pytest.mark.parametrize("mode", ["cached", "dense"])
def test_head_dim_256_paged_fp8k_bf16v_tuned(G, mode):
    """head_dim 256 paged fp8 K beside a bf16 V with a scalar k_scale (the
    reference's paged fp8 cache, paged_eviction.py:354-357): K widened in the
    kernel as bf16(float(fp8) * k_scale), V read as bf16, rows of different
    lengths (the flat layout), the per-wave-prologue kernel."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import paged_pool
    B, hkv, T, d = 3, 2, 10, 256
    k, noise = mixed(B * hkv, T, d, 64, seed=901)
    g = torch.Generator().manual_seed(902)
    v = torch.randn(B * hkv, T * 64, d, generator=g).to(torch.bfloat16)
    q = torch.randn(B * hkv * G, d, generator=g).to(torch.bfloat16)
    ksc = float(k.abs().max()) / 448.0
    k8 = (k / ksc).clamp(-448, 448).to(torch.float8_e4m3fn)
    tab = O.fp8_e4m3fn_table()
    kdeq = np32(torch.from_numpy(tab[k8.view(torch.uint8).numpy()] * np.float32(ksc)).to(torch.bfloat16))
    lens = [T * 64, 7 * 64 + 11, 2 * 64 + 40]
    kc, vc, bt = paged_pool(k8, v, hkv, 16, lens, seed=903)
    row_lens = [lens[r // hkv] for r in range(B * hkv)]
    _, _, _, eh = O.fwht_scores(kdeq.reshape(-1, d), 0.0)
    qn = np.array([O.q_norms(np32(q)[r * G:(r + 1) * G]).max() for r in range(B * hkv)])
    bnd = qn[:, None] * np.sqrt(eh.reshape(B * hkv, T))
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    gate = "none" if mode == "dense" else "cs"
    ref = O.decode_rows(np32(q), kdeq, np32(v), gate=gate, threshold=tau, G=G, lengths=row_lens)
    kv = X.paged_layout(kc.to(DEV), vc.to(DEV), bt.to(DEV), T, keep_mixed=True)
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    kv.k_scale_mode, kv.k_scale = N.OC_KSCALE_DEQUANT, ksc
    e_low, e_high, _, _ = X.score_tiles(kv)
    ng = N.OC_GATE_NONE if mode == "dense" else N.OC_GATE_CS
    nm = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    print(f"head_dim 256 paged fp8 K + bf16 V G={G} {mode}", flush=True)
    r = X.decode(kv, q.to(DEV), G, gate=ng, threshold=tau, mode=nm, scores=(e_low, e_high),
                 out_dtype=torch.float32, want_keep=mode != "dense")
    torch.cuda.synchronize()
    if mode != "dense":
        keep = r.keep.cpu().numpy().astype(bool)
        for row in range(B * hkv):
            nt = -(-row_lens[row] // 64)
            assert np.array_equal(keep[row, :nt], ref["keep"][row, :nt]), row
    assert_out(r.out, ref["out"], "fp8", f"head_dim 256 tuned paged fp8 K + bf16 V G={G} {mode}")


# ------------------------------------------------ head_dim 32, tuned kernels

def _d32_case(rows, T, G, dt, seed):
    k, noise = mixed(rows, T, 32, 64, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    v = torch.randn(rows, T * 64, 32, generator=g)
    q = torch.randn(rows * G, 32, generator=g)
    kd, vd, qd = (x.to(TORCH_DT[dt]).to(DEV) for x in (k, v, q))
    return kd, vd, qd, noise


def _cs_tau_d(qd, kd, noise, G):
    rows, d = kd.shape[0], kd.shape[-1]
    _, _, _, eh = O.fwht_scores(np32(kd).reshape(-1, d), 0.0)
    eh = eh.reshape(rows, -1)
    qn = np.array([O.q_norms(np32(qd)[r * G:(r + 1) * G]).max() for r in range(rows)])
    b = qn[:, None] * np.sqrt(eh)
    return float(0.5 * (b[~noise.numpy()].max() + b[noise.numpy()].min()))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 8, 12])
@pytest.mark.parametrize("gate", ["cs", "zeta", "mask", "none", "cs_single_pass", "zeta_single_pass"])
def test_head_dim_32_tuned_kernel(dt, G, gate):
    """head_dim 32, 64-token tiles, 16-bit K/V with q of K's type, on the
    matrix-core kernels of head_dim 64 / 128 (8-wave workgroups, a 4 KiB V
    slot per wave): the cached score- or mask-gated decode and the dense
    decode on the per-wave-prologue kernel (splits_per_group = 2; G = 12 is
    two head chunks, the general kernel), the single-pass gates on the
    general one; against the oracle, and against the same decode forced onto
    the portable kernels."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T = 3, 12
    kd, vd, qd, noise = _d32_case(rows, T, G, dt, seed=19 * G + 5 * len(gate))
    kv = X.rows_layout(kd, vd)
    q32, k32, v32 = np32(qd), np32(kd), np32(vd)
    tmask = None
    single = gate.endswith("_single_pass")
    gate = gate.replace("_single_pass", "")
    if gate == "cs":
        thr, ng = _cs_tau_d(qd, kd, noise, G), N.OC_GATE_CS
    elif gate == "zeta":
        thr, ng = 5.0, N.OC_GATE_ZETA
    elif gate == "mask":
        thr, ng = 0.0, N.OC_GATE_MASK
        tmask = (torch.rand(rows, T, generator=torch.Generator().manual_seed(G)) < 0.5).to(torch.uint8)
        tmask[:, 0] = 1
    else:
        thr, ng = 0.0, N.OC_GATE_NONE
    if gate == "mask":
        keep = tmask.bool().numpy()
        ref = np.zeros((rows * G, 32), dtype=np.float32)
        for r in range(rows):
            sel = np.repeat(keep[r], 64)
            for h in range(G):
                ref[r * G + h] = O.dense_decode(q32[r * G + h:r * G + h + 1], k32[r:r + 1, sel], v32[r:r + 1, sel])[0]
    else:
        res = O.decode_rows(q32, k32, v32, gate="none" if gate == "none" else gate, threshold=thr, G=G)
        ref, keep = res["out"], res["keep"]
        if gate != "none":
            assert np.array_equal(keep, noise.numpy() if gate == "cs" else ~noise.numpy())
    e_low, e_high, _, _ = X.score_tiles(kv)
    mode = N.OC_MODE_SINGLE_PASS if (gate == "none" or single) else N.OC_MODE_CACHED
    outs = {}
    for portable in (0, 1):
        print(f"head_dim 32 {dt} G={G} gate={gate} single={single} portable={portable}", flush=True)
        r = X.decode(kv, qd, G, gate=ng, threshold=thr, mode=mode, scores=(e_low, e_high), num_splits=4,
                     splits_per_group=2, out_dtype=TORCH_DT[dt], want_keep=gate != "none",
                     tile_mask=None if tmask is None else tmask.to(DEV), portable=portable)
        torch.cuda.synchronize()
        if gate != "none":
            assert np.array_equal(r.keep.cpu().numpy().astype(bool), keep), portable
        assert_out(r.out, ref, dt, f"head_dim 32 {'portable' if portable else 'tuned'} {dt} G={G} {gate}"
                                   f"{' single pass' if single else ''}")
        outs[portable] = np32(r.out)
    # the two kernels agree to the output type's rounding
    assert np.max(np.abs(outs[0] - outs[1])) <= {"bf16": 1.6e-2, "f16": 2e-3}[dt]


def test_head_dim_32_routing_and_full_row():
    """With the automatic split grouping, head_dim 32 bf16 cached decodes take
    several splits per workgroup (the tuned kernels' grouping: fewer
    partials than splits) while the same call forced portable keeps one
    split per workgroup; the tuned kernels' output on 8 rows x 10240 tokens
    (160 tiles) matches the oracle, cached and dense, with the fused merge
    over one head (64 merge slices of 512 threads) and over four."""
    import ctypes
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T = 8, 160
    lib = N.lib()
    for G in (1, 4):
        kd, vd, qd, noise = _d32_case(rows, T, G, "bf16", seed=320 + G)
        kv = X.rows_layout(kd, vd)
        tau = _cs_tau_d(qd, kd, noise, G)
        e_low, e_high, _, _ = X.score_tiles(kv)
        P = X.auto_num_splits(T, qd.device)
        groups = {}
        for portable in (0, 1):
            p = N.OcDecodeParams()
            p.kv = kv.struct()
            p.q, p.q_dtype, p.G, p.q_row_stride = qd.data_ptr(), N.OC_BF16, G, qd.stride(0)
            p.gate, p.mode, p.threshold = N.OC_GATE_CS, N.OC_MODE_CACHED, tau
            p.score_e_low, p.score_e_high, p.score_row_stride = e_low.data_ptr(), e_high.data_ptr(), e_high.stride(0)
            p.num_splits, p.out_dtype, p.portable = P, N.OC_BF16, portable
            groups[portable] = lib.oc_decode_num_groups(ctypes.byref(p))
        assert groups[1] == P and groups[0] < P, (P, groups)
        q32, k32, v32 = np32(qd), np32(kd), np32(vd)
        for gate, ng, mode in (("cs", N.OC_GATE_CS, N.OC_MODE_CACHED), ("none", N.OC_GATE_NONE, N.OC_MODE_SINGLE_PASS)):
            ref = O.decode_rows(q32, k32, v32, gate=gate, threshold=tau, G=G)
            print(f"head_dim 32 full row G={G} {gate}", flush=True)
            r = X.decode(kv, qd, G, gate=ng, threshold=tau, mode=mode, scores=(e_low, e_high), num_splits=P,
                         out_dtype=torch.bfloat16, want_keep=gate == "cs")
            torch.cuda.synchronize()
            if gate == "cs":
                assert np.array_equal(r.keep.cpu().numpy().astype(bool), ref["keep"])
            assert_out(r.out, ref["out"], "bf16", f"head_dim 32 tuned full row G={G} {gate}")


def test_head_dim_32_partials_single_pass():
    """return_partials at head_dim 32 (one workgroup per logical split, the
    general matrix-core kernel, single-pass CS gate): every split's (m, l,
    acc) against the oracle's, and the merged output."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T, G = 2, 9, 4
    kd, vd, qd, noise = _d32_case(rows, T, G, "bf16", seed=32)
    kv = X.rows_layout(kd, vd)
    tau = _cs_tau_d(qd, kd, noise, G)
    print("head_dim 32 partials", flush=True)
    res = X.decode(kv, qd, G, gate=N.OC_GATE_CS, threshold=tau, num_splits=4, out_dtype=torch.float32,
                   want_partials=True, want_keep=True)
    torch.cuda.synchronize()
    ref = O.decode_rows(np32(qd), np32(kd), np32(vd), gate="cs", threshold=tau, G=G, num_splits=4,
                        want_partials=True)
    assert np.array_equal(res.keep.cpu().numpy().astype(bool), ref["keep"])
    pm, pl, pacc = (np32(t) for t in res.partials)
    assert np.array_equal(pm == np.float32(-1e9), ref["M"] == np.float32(-1e9))
    np.testing.assert_allclose(pm, ref["M"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pl, ref["L"], rtol=1e-5, atol=1e-6)
    # about 16 bits of each p in the matrix-core p.V (see the head_dim 256 case)
    scale = float(np.abs(ref["ACC"]).max())
    np.testing.assert_allclose(pacc, ref["ACC"], rtol=1e-5, atol=1e-5 * max(1.0, scale))
    assert_out(res.out, ref["out"], "f32", "head_dim 32 tuned partials merged")


@pytest.mark.parametrize("bs", [16, 64])
@pytest.mark.parametrize("mode", ["cached", "single_pass", "dense"])
def test_head_dim_32_paged_tuned(bs, mode):
    """head_dim 32 paged f16 decode on the matrix-core kernels: 3 sequences x
    2 kv heads, G = 4, row lengths with partial tail tiles (the flat layout
    of rows of different lengths for the cached and dense decodes), a
    shuffled pool with 16- and 64-token pages; the Cauchy-Schwarz gate at a
    calibrated tau, against the oracle's decode over the rows' lengths."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.workloads import paged_pool
    B, hkv, G, T, d = 3, 2, 4, 14, 32
    k, noise = mixed(B * hkv, T, d, 64, seed=32 + bs)
    g = torch.Generator().manual_seed(3 * bs)
    v = torch.randn(B * hkv, T * 64, d, generator=g)
    q = torch.randn(B * hkv * G, d, generator=g)
    k, v, q = (x.to(torch.float16) for x in (k, v, q))
    lens = [T * 64, 9 * 64 + 37, 3 * 64 + 5]
    kc, vc, bt = paged_pool(k, v, hkv, bs, lens, seed=bs + 1)
    row_lens = [lens[r // hkv] for r in range(B * hkv)]
    k32, v32, q32 = np32(k), np32(v), np32(q)
    _, _, _, eh = O.fwht_scores(k32.reshape(-1, d), 0.0)
    eh = eh.reshape(B * hkv, T)
    qn = np.array([O.q_norms(q32[r * G:(r + 1) * G]).max() for r in range(B * hkv)])
    bnd = qn[:, None] * np.sqrt(eh)
    tau = float(0.5 * (bnd[~noise.numpy()].max() + bnd[noise.numpy()].min()))
    gate = "none" if mode == "dense" else "cs"
    ref = O.decode_rows(q32, k32, v32, gate=gate, threshold=tau, G=G, lengths=row_lens)
    kv = X.paged_layout(kc.to(DEV), vc.to(DEV), bt.to(DEV), T)
    kv.lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    e_low, e_high, _, _ = X.score_tiles(kv)
    ng = N.OC_GATE_NONE if mode == "dense" else N.OC_GATE_CS
    nm = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    print(f"head_dim 32 paged bs={bs} {mode}", flush=True)
    r = X.decode(kv, q.to(DEV), G, gate=ng, threshold=tau, mode=nm, scores=(e_low, e_high),
                 out_dtype=torch.float32, want_keep=mode != "dense")
    torch.cuda.synchronize()
    if mode != "dense":
        keep = r.keep.cpu().numpy().astype(bool)
        for row in range(B * hkv):
            nt = -(-row_lens[row] // 64)
            assert np.array_equal(keep[row, :nt], ref["keep"][row, :nt]), row
    assert_out(r.out, ref["out"], "f32", f"head_dim 32 tuned paged bs={bs} {mode}")


@pytest.mark.parametrize("scale", ["q_fold", "tile"])
@pytest.mark.parametrize("mode", ["cached", "single_pass", "dense"])
def test_head_dim_32_scale_modes(scale, mode):
    """head_dim 32 bf16 on the matrix-core kernels with a scalar k_scale folded
    into q (the reference's semantics) or per-(row, tile) K and V scales: keep
    flags and outputs equal, to the output's rounding, to the same call on the
    portable kernels; the tile-scale outputs also against the oracle on the
    scaled values (the zeta gate, whose ratio the tile scales leave as it is)."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    rows, T, G, d = 3, 12, 4, 32
    k, noise = mixed(rows, T, d, 64, seed=3200 + len(mode) + len(scale))
    g = torch.Generator().manual_seed(3201)
    v = torch.randn(rows, T * 64, d, generator=g)
    q = torch.randn(rows * G, d, generator=g)
    kd, vd, qd = (x.to(torch.bfloat16).to(DEV) for x in (k, v, q))
    kv = X.rows_layout(kd, vd)
    ks = vs = None
    if scale == "tile":
        ks = 0.5 + torch.rand(rows, T, generator=g)
        vs = 0.5 + torch.rand(rows, T, generator=g)
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(ks.to(DEV), rows, T, DEV)
        kv.v_scale_mode, kv.v_scales = X.vscale_mode(vs.to(DEV), rows, T, DEV)
    else:
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(1.25, rows, T, DEV)
    e_low, e_high, _, _ = X.score_tiles(kv)
    ng = N.OC_GATE_NONE if mode == "dense" else N.OC_GATE_ZETA
    nm = N.OC_MODE_CACHED if mode == "cached" else N.OC_MODE_SINGLE_PASS
    outs, keeps = {}, {}
    for portable in (0, 1):
        print(f"head_dim 32 {scale} {mode} portable={portable}", flush=True)
        r = X.decode(kv, qd, G, gate=ng, threshold=5.0, mode=nm, scores=(e_low, e_high), num_splits=4,
                     splits_per_group=2, out_dtype=torch.float32, want_keep=mode != "dense", portable=portable)
        torch.cuda.synchronize()
        outs[portable] = np32(r.out)
        if mode != "dense":
            keeps[portable] = r.keep.cpu().numpy().astype(bool)
    if mode != "dense":
        assert np.array_equal(keeps[0], keeps[1])
        assert np.array_equal(keeps[0], ~noise.numpy())
    assert np.max(np.abs(outs[0] - outs[1])) <= 2e-3, scale
    if scale == "tile":
        ref = O.decode_rows(np32(qd), np32(kd), np32(vd), gate="none" if mode == "dense" else "zeta", threshold=5.0,
                            G=G, k_scales=ks.numpy(), v_scales=vs.numpy())
        assert_out(outs[0], ref["out"], "f32", f"head_dim 32 tuned tile scales {mode}")
