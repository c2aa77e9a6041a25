"""64-point Walsh-Hadamard tile scoring on MI355X.

Drop-in for the reference module of the same name
(src/orthocache_gpu/triton_kernels/fwht_fused_prototype.py): the constants,
`generate_walsh_matrix` and `triton_fwht_eviction` keep their names and
meaning; the transform and the band energies run in liborthocache_hip
(oc_score_tiles / oc_fwht_tiles).  The module name is kept for import
compatibility; nothing here uses Triton.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _launch as X

TILE_SIZE = 64  # tokens per spectral tile (fwht_fused_prototype.py:42)

# 64-point bands in natural (Sylvester) row order (fwht_fused_prototype.py:44-50)
BAND_DC_64 = 0
BAND_LOW_64 = (1, 8)
BAND_MID_64 = (8, 32)
BAND_HIGH_64 = (32, 64)


def generate_walsh_matrix(n: int) -> torch.Tensor:
    """n x n Sylvester Hadamard matrix scaled by 1/sqrt(n), float32 on CPU:
    H_{2m} = [[H, H], [H, -H]] (fwht_fused_prototype.py:57-80)."""
    assert n > 0 and (n & (n - 1)) == 0, f"n must be a power of 2, got {n}"
    h = torch.tensor([[1.0]], dtype=torch.float32)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], dim=1), torch.cat([h, -h], dim=1)], dim=0)
    return h / (n ** 0.5)


def _check_tiles(keys: torch.Tensor, tile_size: int) -> int:
    assert keys.ndim == 2, f"keys must be 2D (tokens, head_dim), got {keys.shape}"
    num_tokens = keys.shape[0]
    num_tiles = num_tokens // tile_size
    assert num_tokens == num_tiles * tile_size, (
        f"seq_len {num_tokens} not divisible by tile_size {tile_size}")
    if tile_size != TILE_SIZE:
        raise NotImplementedError(f"the HIP kernels implement {TILE_SIZE}-token tiles only, got {tile_size}")
    return num_tiles


def triton_fwht_eviction(
    keys: torch.Tensor,
    zeta_max: float,
    tile_size: int = TILE_SIZE,
    return_zeta: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Per-tile eviction mask from the spectral decay ratio.

    keys (num_tiles*64, head_dim) on the GPU.  Returns (mask, zeta): mask is
    bool (num_tiles,) with True = retain (zeta <= zeta_max), zeta the float32
    ratio e_high/(e_low+1e-6) when return_zeta, else None
    (fwht_fused_prototype.py:255-322).
    """
    num_tiles = _check_tiles(keys, tile_size)
    X.require_gpu(keys)
    kv = X.rows_layout(keys.unsqueeze(0), None)
    kv.num_tiles = num_tiles
    _, _, zeta, keep = X.score_tiles(kv, zeta_max, want_zeta=return_zeta, want_keep=True)
    mask = keep[0, :num_tiles].bool()
    return mask, (zeta[0, :num_tiles] if return_zeta else None)


def score_tiles(keys: torch.Tensor, zeta_max: float = 0.0, k_scale=None):
    """Band energies of every 64-token tile of (rows, S, d) keys (or (S, d)).

    Returns a TileScores with e_low, e_high, zeta (rows, T) float32 and keep
    (rows, T) bool for zeta_max.  These are the cached scores that the
    decode entry points accept as `score_cache=` (mode='cached'): a tile's
    scores depend only on its keys, so they are computed once when the tile
    is complete and reused by every later decode step.
    `k_scale`: optional (rows, T) float32 per-tile K scales (fp8 caches).
    """
    squeeze = keys.ndim == 2
    if squeeze:
        keys = keys.unsqueeze(0)
    assert keys.ndim == 3, f"keys must be (rows, S, d) or (S, d), got {tuple(keys.shape)}"
    X.require_gpu(keys)
    kv = X.rows_layout(keys, None)
    if k_scale is not None:
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, kv.num_rows, kv.num_tiles, keys.device)
        if kv.k_scale_mode != X.N.OC_KSCALE_TILE:
            kv.k_scale_mode, kv.k_scale = X.N.OC_KSCALE_NONE, 1.0
    e_low, e_high, zeta, keep = X.score_tiles(kv, zeta_max)
    return TileScores(e_low[:, :kv.num_tiles], e_high[:, :kv.num_tiles], zeta[:, :kv.num_tiles],
                      keep[:, :kv.num_tiles].bool())


class TileScores:
    """Cached per-(row, tile) spectral scores (see score_tiles)."""

    def __init__(self, e_low, e_high, zeta=None, keep=None):
        self.e_low, self.e_high, self.zeta, self.keep = e_low, e_high, zeta, keep

    def as_pair(self):
        return self.e_low, self.e_high


def fwht_tiles(keys: torch.Tensor) -> torch.Tensor:
    """The full transform X = W64 @ K_tile of every tile of (S, d) or
    (rows, S, d) keys, float32 (rows, T, 64, d) (or (T, 64, d))."""
    squeeze = keys.ndim == 2
    if squeeze:
        keys = keys.unsqueeze(0)
    X.require_gpu(keys)
    kv = X.rows_layout(keys, None)
    out = X.fwht_tiles(kv)
    return out[0] if squeeze else out
