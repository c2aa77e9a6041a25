"""GPU parity of the score-cache maintenance, the O(1) decode gate and the
mask-given attention: oc_band_norms (SpectralNormCache), oc_score_tile_range
(TileScores.update), oc_decode_gate, oc_q_high_norms, oc_apply_tile_mask and
oc_decode with OC_GATE_MASK (block-sparse / indirect attention) against the
oracle.

Bars: band norms and q norms within 4 float32 ulp of the oracle (the
summation order differs); masks bit-exact on data whose gate products are
away from the threshold; scores from the append path bit-identical to a
full scoring pass (same kernel); masked logits exact.
"""

import numpy as np
import pytest
import torch

from oracle import orthocache_oracle as O
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


def _keys(rows, tiles, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((rows, tiles * 64, d), generator=g) + 0.5
    k[:, ::7] *= 3.0
    return k.to(TORCH_DT[dtype]) if dtype != "fp8" else (k * 20).clamp(-448, 448).to(torch.float8_e4m3fn)


def _decoded(k):
    if k.dtype == torch.float8_e4m3fn:
        return O.fp8_e4m3fn_table()[k.view(torch.uint8).numpy()]
    return np32(k)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16", "fp8"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("band", [(48, 64), (32, 64), (1, 8), (0, 64)])
def test_populate_from_keys_vs_oracle(dtype, d, band):
    from orthocache_gpu import generate_walsh_matrix
    from orthocache_gpu.norm_cache import SpectralNormCache
    k = _keys(3, 9, d, dtype, seed=d + band[0])
    cache = SpectralNormCache(4, 12, torch.device(DEV))
    cache.populate_from_keys(k.to(DEV), generate_walsh_matrix(64).to(DEV), high_start=band[0], high_end=band[1])
    ref = O.band_norms(_decoded(k), *band)
    got = np32(cache.cache)
    np.testing.assert_allclose(got[:3, :9], ref, rtol=4 * 2.0 ** -23, atol=0)
    assert (got[3] == 0).all() and (got[:, 9:] == 0).all()
    assert cache.valid_tiles.cpu().tolist() == [9, 9, 9, 0]
    assert cache.is_populated


def test_update_prefill_and_append_path():
    from orthocache_gpu import generate_walsh_matrix
    from orthocache_gpu.norm_cache import SpectralNormCache
    w = generate_walsh_matrix(64).to(DEV)
    k = _keys(2, 10, 128, "bf16", seed=3).to(DEV)
    full = SpectralNormCache(2, 16, torch.device(DEV)).populate_from_keys(k, w)
    c = SpectralNormCache(2, 16, torch.device(DEV))
    c.update_prefill(1, 5, k[1, 5 * 64:6 * 64], w, 48, 64)
    c.update_prefill(1, 2, k[1, 2 * 64:3 * 64], w, 48, 64)
    assert c.valid_tiles.cpu().tolist() == [0, 6]
    assert c.get_norm(1, 5) == full.get_norm(1, 5) and c.get_norm(1, 2) == full.get_norm(1, 2)
    assert c.get_norm(1, 3) == 0.0 and c.get_norms_batch(1).shape == (6,)
    # append path: a decode step completed tiles 7 and 8
    c.update_tiles(k, 7, 2)
    assert torch.equal(c.cache[:, 7:9], full.cache[:, 7:9])
    assert c.valid_tiles.cpu().tolist() == [9, 9]
    # with lengths, a tile not yet complete is skipped
    c.update_tiles(k, 9, 1, context_lens=torch.tensor([9 * 64 + 10, 10 * 64], device=DEV))
    assert c.get_norm(0, 9) == 0.0 and c.get_norm(1, 9) == full.get_norm(1, 9)
    # a multiple of the Walsh matrix scales the norms (exactly for powers of
    # two); any other matrix is refused
    c.update_prefill(0, 0, k[0, :64], w * 2, 48, 64)
    assert c.get_norm(0, 0) == 2 * full.get_norm(0, 0)
    with pytest.raises(NotImplementedError):
        c.update_prefill(0, 0, k[0, :64], w.flip(0), 48, 64)


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_tile_scores_append_equals_full_scoring(dtype):
    from orthocache_gpu import TileScores, score_tiles
    k = _keys(3, 11, 128, dtype, seed=9).to(DEV)
    ks = None
    if dtype == "fp8":
        ks = torch.rand((3, 11), generator=torch.Generator().manual_seed(2)).to(DEV) + 0.5
    full = score_tiles(k, zeta_max=5.0, k_scale=ks)
    sc = TileScores.allocate(3, 16, DEV, zeta_max=5.0)
    sc.update(k, 0, 6, k_scale=ks)
    for t in range(6, 11):
        sc.update(k, t, k_scale=ks)  # one tile per decode step
    for name in ("e_low", "e_high", "zeta", "keep"):
        assert torch.equal(getattr(sc, name)[:, :11], getattr(full, name)), name
    assert not sc.e_high[:, 11:].any()


@pytest.mark.parametrize("q_norm", ["spatial", "high"])
@pytest.mark.parametrize("qdtype", ["f32", "bf16"])
def test_decode_gate_vs_oracle(q_norm, qdtype):
    from orthocache_gpu.triton_kernels.decode_gate import decode_gate
    rng = np.random.default_rng(11)
    G, hkv, d, max_tiles, num_tiles = 4, 8, 128, 300, 257
    q = torch.from_numpy(rng.standard_normal((hkv * G, d)).astype(np.float32)).to(TORCH_DT[qdtype])
    nc = rng.uniform(0.0, 50.0, size=(hkv, max_tiles)).astype(np.float32)
    tight = q_norm == "high"
    _, qn_ref = O.decode_gate(np32(q), nc, 0.0, num_tiles, G, tight=tight)
    # a tau whose products stay >= 1e-3 relative away from every decision
    prod = np.sort((qn_ref[:, None] * nc[:, :num_tiles]).ravel())
    gaps = prod[1:] / np.maximum(prod[:-1], 1e-30)
    i = int(np.argmax(gaps[len(gaps) // 4:3 * len(gaps) // 4])) + len(gaps) // 4
    tau = float(np.sqrt(prod[i] * prod[i + 1])) / (64 * d)
    mask_ref, qn_ref = O.decode_gate(np32(q), nc, tau, num_tiles, G, tight=tight)
    mask, qn = decode_gate(q.to(DEV), torch.from_numpy(nc).to(DEV), tau, num_tiles, G, q_norm=q_norm)
    assert mask.dtype == torch.bool and mask.shape == (hkv, max_tiles)
    np.testing.assert_allclose(np32(qn), qn_ref, rtol=4 * 2.0 ** -23)
    assert np.array_equal(mask.cpu().numpy(), mask_ref)
    assert 0 < mask_ref.sum() < hkv * num_tiles


def test_q_high_norms_vs_oracle():
    from orthocache_gpu.triton_kernels.decode_gate import compute_q_high_norm_exact
    rng = np.random.default_rng(12)
    for shape, low_band in (((2, 32, 128), 8), ((7, 64), 8), ((5, 128), 16)):
        q = rng.standard_normal(shape).astype(np.float32)
        got = compute_q_high_norm_exact(torch.from_numpy(q).to(DEV), low_band)
        assert got.shape == shape[:-1]
        np.testing.assert_allclose(np32(got), O.q_high_norm_exact(q, low_band), rtol=8 * 2.0 ** -23, atol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_apply_decode_mask_exact(dtype):
    from orthocache_gpu.triton_kernels.decode_gate import apply_decode_mask, apply_decode_mask_vectorized
    rng = np.random.default_rng(13)
    G, hkv, s_len = 4, 3, 64 * 9 + 21
    logits = torch.from_numpy(rng.standard_normal((hkv * G, 1, s_len)).astype(np.float32)).to(TORCH_DT[dtype])
    mask = torch.from_numpy(rng.random((hkv, 12)) < 0.4)
    ref = O.apply_decode_mask(np32(logits), mask.numpy(), G)
    for fn in (apply_decode_mask, apply_decode_mask_vectorized):
        got = fn(logits.clone().to(DEV), mask.to(DEV), G)
        assert np.array_equal(np32(got), ref)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("block_size", [512, 128, 64])
def test_block_sparse_attention_vs_oracle(dtype, block_size):
    from orthocache_gpu.triton_kernels import triton_block_sparse_attention
    g = torch.Generator().manual_seed(block_size)
    n_blocks, d = 24, 128
    q = torch.randn((1, d), generator=g).to(TORCH_DT[dtype])
    k = torch.randn((n_blocks * block_size, d), generator=g).to(TORCH_DT[dtype])
    v = torch.randn((n_blocks * block_size, d), generator=g).to(TORCH_DT[dtype])
    for mask in (torch.rand(n_blocks, generator=g) < 0.4, torch.ones(n_blocks, dtype=torch.bool),
                 torch.zeros(n_blocks, dtype=torch.bool)):
        out = triton_block_sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV), block_size)
        assert out.dtype == q.dtype and out.shape == (1, d)
        ref = O.block_sparse_attention(np32(q), np32(k), np32(v), mask.numpy(), block_size)
        assert_out(out, ref, dtype, f"block sparse {dtype} bs={block_size}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_indirect_attention_vs_oracle(dtype):
    from orthocache_gpu.triton_kernels import triton_indirect_attention
    g = torch.Generator().manual_seed(7)
    n_blocks, d, bs = 20, 128, 512
    q = torch.randn((1, d), generator=g).to(TORCH_DT[dtype])
    k = torch.randn((n_blocks * bs + 100, d), generator=g).to(TORCH_DT[dtype])  # a partial block at the end
    v = torch.randn((n_blocks * bs + 100, d), generator=g).to(TORCH_DT[dtype])
    idx = torch.randperm(n_blocks, generator=g)[:9].to(torch.int32)
    out = triton_indirect_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), 7, bs)
    ref = O.indirect_attention(np32(q), np32(k), np32(v), idx.numpy(), 7, bs)
    assert_out(out, ref, dtype, f"indirect {dtype}")
    zero = triton_indirect_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), 0, bs)
    assert not zero.any()
    with pytest.raises(ValueError, match="block index"):
        triton_indirect_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor([3, 99], dtype=torch.int32,
                                                                                 device=DEV), 2, bs)
