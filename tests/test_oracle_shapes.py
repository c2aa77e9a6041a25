"""CPU tests that pin the oracle at head dims other than 64 / 128 and tiles
other than 64 tokens (no GPU).

The reference asserts only that head_dim and tile_size are powers of two
(fused_eviction.py:609-610, gqa_eviction.py:551-552, paged_eviction.py:
345-347) and keeps its bands at the spectrum rows [1, 8) and [32, 64),
clipped to the tile (fused_eviction.py:424-427).  The oracle's functions
take tile_size and any head_dim; here they are held to:
* the reference's own outputs at such shapes (tests/golden/shapes_*,
  written by tests/golden/make_golden_shapes.py);
* the textbook butterfly (Walsh matrices of every size up to 256);
* what the band clipping fixes: no high band below 33-token tiles (zeta 0,
  every tile kept by the zeta gate, every tile evicted by the
  Cauchy-Schwarz gate at tau >= 0), no low band for 1-token tiles;
* a planted mistake (the bands scaled to the tile size) that must fail.
"""

import json
import os

import numpy as np
import pytest

from oracle import orthocache_oracle as O
from tests import golden_io

F32 = np.float32


def _cases():
    with open(os.path.join(golden_io.GOLDEN_DIR, "MANIFEST_shapes.json")) as f:
        return json.load(f)["cases"]


def _out_tol(dtype):
    return {"f32": 2e-6, "f16": 2e-3, "bf16": 8e-3}[dtype]


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 32, 128, 256])
def test_walsh_matrix_every_size(n):
    w = O.walsh_matrix(n).astype(np.float64)
    assert np.allclose(w @ w.T, np.eye(n), atol=1e-6)
    assert np.allclose(w, O.fwht64_butterfly(np.eye(n)), atol=1e-7)  # the textbook butterfly, any size


def test_manifest_lists_every_shape_case():
    names = _cases()
    assert len(names) == 17
    for n in names:
        assert os.path.exists(os.path.join(golden_io.GOLDEN_DIR, n + ".npz")), n


@pytest.mark.parametrize("ts", [16, 32, 128, 256])
def test_golden_scores_other_tile_sizes(ts):
    raw, dec, dt, meta, params, _ = golden_io.load(f"shapes_fwht_ts{ts}")
    keep, zeta, e_low, e_high = O.fwht_scores(dec["keys"], params["zeta_max"], tile_size=ts)
    assert np.array_equal(keep, dec["mask"].astype(bool))
    assert np.allclose(zeta, dec["zeta"], rtol=1e-5, atol=1e-6)
    if ts <= 32:
        assert not e_high.any() and not zeta.any() and keep.all()  # no high band
    else:
        assert 0 < keep.sum() < keep.size


@pytest.mark.parametrize("name", ["shapes_v1_d32", "shapes_v1_ts128"])
def test_golden_v1_shapes(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m = O.fused_v1(dec["q"], dec["keys"], dec["values"], params["zeta_max"], tile_size=params["tile_size"],
                        return_mask=True)
    for k in ("tiles_retained", "tiles_evicted", "eviction_rate"):
        assert m[k] == meta[k]
    assert np.array_equal(m["eviction_mask"], meta["eviction_mask"])
    assert np.max(np.abs(O.round_to(out, dt["out"]) - dec["out"])) <= _out_tol(dt["out"])


@pytest.mark.parametrize("name", ["shapes_v2_d256_bf16", "shapes_v2_d32_f16", "shapes_v2_d16_ts16_f32",
                                  "shapes_v2_ts32_f32", "shapes_v2_ts128_bf16"])
def test_golden_v2_shapes(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.fused_v2(dec["q"], dec["keys"], dec["values"], params["zeta_max"],
                              tile_size=params["tile_size"])
    assert {k: m[k] for k in meta} == meta
    assert np.max(np.abs(O.round_to(out, dt["out"]) - dec["out"])) <= _out_tol(dt["out"])
    if params["tile_size"] <= 32:
        assert mask.all()


@pytest.mark.parametrize("name", ["shapes_v3_d256_f32", "shapes_v3_ts128_bf16", "shapes_v3_ts32_f32"])
def test_golden_v3_shapes(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.gqa_v3(dec["q"], dec["keys"], dec["values"], params["tau"], params["G"],
                            tile_size=params["tile_size"])
    assert m == meta
    assert np.max(np.abs(O.round_to(out, dt["out"]) - dec["out"])) <= _out_tol(dt["out"])
    if params["tile_size"] <= 32:
        assert not mask.any() and not out.any()  # the empty high band evicts every tile


@pytest.mark.parametrize("name", ["shapes_paged_d256", "shapes_paged_ts128", "shapes_paged_d32_ts32"])
def test_golden_paged_shapes(name):
    raw, dec, dt, meta, params, _ = golden_io.load(name)
    out, m, mask = O.paged(dec["q"], dec["k_cache"], dec["v_cache"], raw["block_tables"], params["zeta_max"],
                           tile_size=params["tile_size"])
    assert m == meta == {}
    assert np.max(np.abs(O.round_to(out, dt["out"]) - dec["out"])) <= _out_tol(dt["out"])


def test_band_clipping_closed_forms():
    """A 128-token tile whose spectrum sits on rows 64..127 only has no band
    energy at all (both bands end by row 63); one on row 40 only has all its
    energy in the high band; a 1-token tile has neither band."""
    rng = np.random.default_rng(5)
    w = O.walsh_matrix(128)
    c = np.zeros((128, 32), dtype=F32)
    c[64:] = rng.standard_normal((64, 32)).astype(F32)
    el, eh = O.tile_energies((w.T @ c).astype(F32), w)
    assert abs(float(el)) < 1e-3 and abs(float(eh)) < 1e-3
    c = np.zeros((128, 32), dtype=F32)
    c[40] = rng.standard_normal(32).astype(F32)
    el, eh = O.tile_energies((w.T @ c).astype(F32), w)
    assert abs(float(el)) < 1e-4 and np.isclose(float(eh), float(np.sum(c[40].astype(np.float64) ** 2)), rtol=1e-5)
    el, eh = O.tile_energies(rng.standard_normal((1, 8)).astype(F32), O.walsh_matrix(1))
    assert float(el) == 0.0 and float(eh) == 0.0


def test_planted_band_scaling_is_caught():
    """Bands scaled to the tile size (rows [TS/32, TS/8) and [TS/2, TS), a
    plausible misreading) change the 128-token golden masks."""
    raw, dec, dt, meta, params, _ = golden_io.load("shapes_fwht_ts128")
    keys = dec["keys"]
    w = O.walsh_matrix(128)
    tiles = keys.reshape(-1, 128, keys.shape[1])
    spec = np.matmul(w[None], tiles)
    eps = np.sum(spec * spec, axis=2, dtype=F32)
    zeta_wrong = eps[:, 64:128].sum(1) / (eps[:, 4:16].sum(1) + F32(1e-6))
    assert not np.array_equal(zeta_wrong <= 5.0, dec["mask"].astype(bool)) or \
        not np.allclose(zeta_wrong, dec["zeta"], rtol=1e-3)
