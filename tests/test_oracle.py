"""CPU tests that pin the oracle (no GPU).

Every oracle function is checked against something that does not restate its
own formula: the reference's golden vectors (tests/golden/), the textbook
butterfly, closed forms of the band energies, integer known-answer tiles,
float64 brute force, and planted mistakes that must be caught.
"""

import math

import numpy as np
import pytest

from oracle import orthocache_oracle as O
from tests import golden_io

RNG = np.random.default_rng(0)
F32 = np.float32


def _int_tile(rng, lo=-4, hi=4, d=128):
    return rng.integers(lo, hi + 1, size=(64, d)).astype(F32)


# ---------------------------------------------------------------- Walsh matrix

def test_walsh_closed_form_and_properties():
    w = O.walsh_matrix(64)
    i = np.arange(64)
    pc = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    assert np.array_equal(w, ((-1.0) ** pc / 8.0).astype(F32))
    assert np.array_equal(w, w.T)
    assert np.allclose(w @ w.T, np.eye(64), atol=1e-6)
    assert np.all(w[0] == F32(0.125))
    for n in (2, 4, 8, 16, 32, 128):
        wn = O.walsh_matrix(n).astype(np.float64)
        assert np.allclose(wn @ wn.T, np.eye(n), atol=1e-6)


def test_band_boundaries_cover_spectrum():
    assert 1 + (O.BAND_LOW_64[1] - O.BAND_LOW_64[0]) + (O.BAND_HIGH_64[0] - O.BAND_LOW_64[1]) \
        + (O.BAND_HIGH_64[1] - O.BAND_HIGH_64[0]) == 64


# ---------------------------------------------------------------- FWHT / energies

def test_matmul_equals_butterfly():
    k = RNG.standard_normal((64, 128)).astype(F32)
    w = O.walsh_matrix(64).astype(np.float64)
    assert np.allclose(w @ k.astype(np.float64), O.fwht64_butterfly(k), atol=1e-12)


def _closed_forms(k):
    k = k.astype(np.float64)
    e_high = 0.5 * np.sum((k[:32] - k[32:]) ** 2)
    s_r = np.stack([k[r::8].sum(axis=0) for r in range(8)])
    e_low = np.sum(s_r ** 2) / 8.0 - np.sum(k.sum(axis=0) ** 2) / 64.0
    return e_low, e_high


@pytest.mark.parametrize("seed", range(5))
def test_energies_match_closed_forms(seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((64, 128)).astype(F32) * (seed + 1)
    el, eh = O.tile_energies(k, O.walsh_matrix())
    cl, ch = _closed_forms(k)
    assert math.isclose(el, cl, rel_tol=2e-5)
    assert math.isclose(eh, ch, rel_tol=2e-5)


@pytest.mark.parametrize("seed", range(8))
def test_integer_known_answer_tiles_exact(seed):
    """Integer entries in [-4, 4]: every coefficient (n/8), square and partial
    sum is a multiple of 1/64 below 2^17, hence exact in float32 in any
    summation order.  The oracle must equal the float64 closed forms bit for
    bit, and so must zeta."""
    rng = np.random.default_rng(100 + seed)
    k = _int_tile(rng)
    el, eh = O.tile_energies(k, O.walsh_matrix())
    cl, ch = _closed_forms(k)
    assert float(el) == cl and float(eh) == ch
    assert O.zeta_of(el, eh) == F32(F32(ch) / F32(F32(cl) + F32(1e-6)))
    spec = O.fwht64_butterfly(k)
    assert float(np.sum(spec[32:] ** 2)) == ch


def test_planted_mistakes_are_caught():
    """Plausible slips in the oracle (a band off by one, transposed operands,
    a dropped 1/8 scale) fail the closed-form pins above."""
    k = _int_tile(np.random.default_rng(7))
    w = O.walsh_matrix()
    cl, ch = _closed_forms(k)
    spec = w @ k
    eps = np.sum(spec * spec, axis=1)
    assert float(np.sum(eps[33:64])) != ch            # band start off by one
    assert float(np.sum(eps[0:8])) != cl              # DC row included
    spec_t = (w @ k[:, :64].T)                        # transposed operand
    assert not np.isclose(float(np.sum((spec_t * spec_t)[32:])),
                          0.5 * np.sum((k[:32, :64] - k[32:, :64]) ** 2))
    spec8 = (w * 8) @ k                                # scale dropped
    assert float(np.sum((spec8 * spec8)[32:])) != ch


# ---------------------------------------------------------------- golden vectors

def _dt_of(dtypes, key):
    dt = dtypes[key]
    return "f32" if dt in ("fp8",) else dt


def test_golden_fwht_scores():
    raw, dec, dt, meta, params, _ = golden_io.load("fwht_scores")
    keep, zeta, _, _ = O.fwht_scores(dec["keys"], params["zeta_max"])
    assert np.array_equal(keep, dec["mask"].astype(bool))
    assert np.allclose(zeta, dec["zeta"], rtol=1e-5, atol=1e-6)


def _out_tol(dtype):
    return {"f32": 2e-6, "f16": 2e-3, "bf16": 8e-3}[dtype]


@pytest.mark.parametrize("name", ["v1_f32", "v1_fp8k_bf16q"])
def test_golden_v1(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = O.fused_v1(dec["q"], dec["keys"], dec["values"], params["zeta_max"],
                        return_mask=True, k_scale=params.get("k_scale", 1.0),
                        q_dtype=dt["q"])
    assert m["tiles_retained"] == meta["tiles_retained"]
    assert m["tiles_evicted"] == meta["tiles_evicted"]
    assert m["eviction_rate"] == meta["eviction_rate"]
    assert np.array_equal(m["eviction_mask"], meta["eviction_mask"])
    got = O.round_to(out, dt["out"])
    assert np.max(np.abs(got - dec["out"])) <= _out_tol(dt["out"])


@pytest.mark.parametrize("name", ["v2_f32", "v2_f16", "v2_bf16"])
def test_golden_v2(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.fused_v2(dec["q"], dec["keys"], dec["values"], params["zeta_max"])
    assert {k: m[k] for k in meta} == meta
    got = O.round_to(out, dt["out"])
    assert np.max(np.abs(got - dec["out"])) <= _out_tol(dt["out"])
    assert 0 < mask.sum() < mask.size


@pytest.mark.parametrize("name", ["v3_f32", "v3_bf16", "v3_fp8k"])
def test_golden_v3(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.gqa_v3(dec["q"], dec["keys"], dec["values"], params["tau"], params["G"],
                            k_scale=params.get("k_scale", 1.0), q_dtype=dt["q"])
    assert m == meta
    got = O.round_to(out, dt["out"])
    assert np.max(np.abs(got - dec["out"])) <= _out_tol(dt["out"])


@pytest.mark.parametrize("name", ["paged_bs16", "paged_bs32", "paged_fp8k"])
def test_golden_paged(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.paged(dec["q"], dec["k_cache"], dec["v_cache"], raw["block_tables"],
                           params["zeta_max"], k_scale=params.get("k_scale", 1.0),
                           q_dtype=dt["q"], k_is_fp8=(dt["k_cache"] == "fp8"))
    assert m == meta == {}
    got = O.round_to(out, dt["out"])
    assert np.max(np.abs(got - dec["out"])) <= _out_tol(dt["out"])


# ---------------------------------------------------------------- brute force

def _retained_dense(q, keys, values, mask):
    """float64 softmax over the tokens of retained tiles only."""
    out = []
    for h in range(keys.shape[0]):
        idx = np.repeat(mask[h], 64)
        if not idx.any():
            out.append(np.zeros(keys.shape[2]))
            continue
        out.append(O.dense_decode(q[h:h + 1], keys[h:h + 1, idx], values[h:h + 1, idx])[0])
    return np.stack(out)


def test_v2_equals_dense_over_retained_tiles():
    _, dec, _, _, params, _ = golden_io.load("v2_f32")
    out, _, mask = O.fused_v2(dec["q"], dec["keys"], dec["values"], params["zeta_max"])
    ref = _retained_dense(dec["q"], dec["keys"], dec["values"], mask)
    assert np.max(np.abs(out - ref)) < 2e-6


def test_zero_and_total_eviction():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 64)).astype(F32)
    k = rng.standard_normal((2, 4 * 64, 64)).astype(F32)
    v = rng.standard_normal((2, 4 * 64, 64)).astype(F32)
    out, m, _ = O.fused_v2(q, k, v, 1e9)
    assert m["tiles_evicted"] == 0
    assert np.max(np.abs(out - O.dense_decode(q, k, v))) < 2e-6
    out0, m0, _ = O.fused_v2(q, k, v, 0.0)
    assert m0["tiles_retained"] == 0 and np.all(out0 == 0)


def test_cs_gate_special_cases():
    """Reference test_gqa_eviction.py:211-308: a constant tile has no high band
    (evicted at tau=0.1), one large-norm query forces retention, all-tiny
    queries allow eviction, tau=0 retains everything."""
    rng = np.random.default_rng(5)
    w = O.walsh_matrix()
    const = np.full((64, 128), 0.5, dtype=F32)
    assert O.tile_energies(const, w)[1] == 0.0
    assert not O.cs_keep(F32(0.0), rng.standard_normal((4, 128)), 0.1)
    k = (rng.standard_normal((64, 128)) * 0.3).astype(F32)
    eh = O.tile_energies(k, w)[1]
    q = np.concatenate([rng.standard_normal((3, 128)) * 1e-3, rng.standard_normal((1, 128)) * 100])
    assert O.cs_keep(eh, q, 1.0)
    assert not O.cs_keep(eh, rng.standard_normal((4, 128)) * 1e-4, 0.1)
    assert O.cs_keep(eh, rng.standard_normal((4, 128)), 0.0)


def test_decode_rows_reduces_to_reference_paths():
    """The generalised oracle equals v2 (zeta, G=1) and v3 (cs) on golden inputs."""
    _, dec, _, meta, params, _ = golden_io.load("v2_f32")
    out, m, mask = O.fused_v2(dec["q"], dec["keys"], dec["values"], params["zeta_max"])
    r = O.decode_rows(dec["q"], dec["keys"], dec["values"], gate="zeta",
                      threshold=params["zeta_max"], G=1)
    assert np.array_equal(r["keep"], mask)
    assert np.max(np.abs(r["out"] - out)) < 2e-6
    _, dec, _, meta, params, _ = golden_io.load("v3_f32")
    out, m, mask = O.gqa_v3(dec["q"], dec["keys"], dec["values"], params["tau"], params["G"])
    r = O.decode_rows(dec["q"], dec["keys"], dec["values"], gate="cs",
                      threshold=params["tau"], G=params["G"])
    assert np.array_equal(r["keep"], mask)
    assert np.max(np.abs(r["out"] - out)) < 2e-6


# ---------------------------------------------------------------- split-K

@pytest.mark.parametrize("t_count,p", [(16, 4), (512, 24), (37, 5), (8, 8)])
def test_interleaved_assignment(t_count, p):
    """Reference test_splitk_kernel.py:300-347: tiles {s + kP} are disjoint,
    cover all tiles and are balanced within one."""
    sets = [set(range(s, t_count, p)) for s in range(p)]
    allt = set()
    for s in sets:
        assert allt.isdisjoint(s)
        allt |= s
    assert allt == set(range(t_count))
    sizes = [len(s) for s in sets]
    assert max(sizes) - min(sizes) <= 1


def test_split_partials_merge_to_single_split():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((4, 64)).astype(F32)
    k = rng.standard_normal((2, 10 * 64, 64)).astype(F32)
    v = rng.standard_normal((2, 10 * 64, 64)).astype(F32)
    one = O.decode_rows(q, k, v, gate="none", threshold=0, G=2)
    for p in (2, 3, 7):
        r = O.decode_rows(q, k, v, gate="none", threshold=0, G=2, num_splits=p,
                          want_partials=True)
        assert np.max(np.abs(r["out"] - one["out"])) < 2e-6
        # float64 merge of the partials equals the float64 dense result
        m, l, acc = r["M"].astype(np.float64), r["L"].astype(np.float64), r["ACC"].astype(np.float64)
        mm = m.max(axis=1, keepdims=True)
        w = np.exp(m - mm)
        merged = (acc * w[..., None]).sum(1) / (l * w).sum(1)[:, None]
        dense = O.dense_decode(q, np.repeat(k, 2, axis=0), np.repeat(v, 2, axis=0))
        assert np.max(np.abs(merged - dense)) < 2e-6


def test_auto_num_splits_formula():
    assert O.auto_num_splits(4, 256) == 1
    assert O.auto_num_splits(128, 256) == 32
    assert O.auto_num_splits(512, 256) == 128
    assert O.auto_num_splits(1024, 256) == 256
    assert O.auto_num_splits(2048, 256) == 256
    assert O.auto_num_splits(3, 256) == 1
    assert O.auto_num_splits(100, None) == 1


def test_context_length_tail_tile():
    """Extension: a partial tail tile is retained and its padding is masked;
    with full-length rows the result equals the unmasked path."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 64)).astype(F32)
    k = rng.standard_normal((1, 4 * 64, 64)).astype(F32)
    v = rng.standard_normal((1, 4 * 64, 64)).astype(F32)
    r = O.decode_rows(q, k, v, gate="zeta", threshold=1e9, G=1, lengths=[150])
    ref = O.dense_decode(q, k[:, :150], v[:, :150])
    assert np.max(np.abs(r["out"] - ref)) < 2e-6
    assert r["keep"][0].tolist() == [True, True, True, False]


def test_fp8_table_and_encoder():
    import torch
    table = O.fp8_e4m3fn_table()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn)
    ref = codes.float().numpy()
    same = (table == ref) | (np.isnan(table) & np.isnan(ref))
    assert same.all()
    x = (RNG.standard_normal(4096) * 50).astype(F32)
    enc = O.fp8_encode(x)
    ref_codes = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(enc, ref_codes)


def test_literal_head_dim_reading_does_not_separate_the_tiles():
    """The config text read with the Walsh rows along head_dim (the literal
    reading) makes every tile white noise along the tokens: zeta centres on
    32/7 for "smooth" and "noise" tiles alike, and zeta_max = 5 evicts a
    label-independent share of both -- why the benchmarks build the tiles
    along the tokens, as the reference's own benchmark does."""
    from orthocache_gpu.workloads import make_kv_literal
    keys, noise = make_kv_literal(8, 64 * 200, 128, seed=3)
    _, zeta = O.fwht_scores(keys.reshape(-1, 128).numpy(), 5.0)[:2]
    zeta, noise = np.asarray(zeta), noise.reshape(-1).numpy()
    for part in (zeta[noise], zeta[~noise]):
        assert abs(float(np.median(part)) - 32 / 7) < 0.3
        assert 0.05 < float((part > 5.0).mean()) < 0.6
