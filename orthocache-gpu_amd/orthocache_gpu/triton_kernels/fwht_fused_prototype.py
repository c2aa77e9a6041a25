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
    X.check_tile_size(tile_size)
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
    kv = X.rows_layout(keys.unsqueeze(0), None, tile_size=tile_size)
    kv.num_tiles = num_tiles
    _, _, zeta, keep = X.score_tiles(kv, zeta_max, want_zeta=return_zeta, want_keep=True)
    mask = keep[0, :num_tiles].bool()
    return mask, (zeta[0, :num_tiles] if return_zeta else None)


def score_tiles(keys: torch.Tensor, zeta_max: float = 0.0, k_scale=None, *, tile_size: int = TILE_SIZE):
    """Band energies of every tile (64 tokens, or `tile_size`) of (rows, S, d)
    keys (or (S, d)).

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
    X.check_tile_size(tile_size)
    kv = X.rows_layout(keys, None, tile_size=tile_size)
    if k_scale is not None:
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, kv.num_rows, kv.num_tiles, keys.device)
        if kv.k_scale_mode != X.N.OC_KSCALE_TILE:
            kv.k_scale_mode, kv.k_scale = X.N.OC_KSCALE_NONE, 1.0
    e_low, e_high, zeta, keep = X.score_tiles(kv, zeta_max)
    return TileScores(e_low[:, :kv.num_tiles], e_high[:, :kv.num_tiles], zeta[:, :kv.num_tiles],
                      keep[:, :kv.num_tiles].bool(), zeta_max=zeta_max, tile_size=tile_size)


class TileScores:
    """Cached per-(row, tile) spectral scores (see score_tiles).

    The append path: `TileScores.allocate` sizes a cache for the longest
    context, the prefill scores its complete tiles with `update`, and each
    decode step that completes a tile rescores only that tile with
    `update(keys, t)` (one small launch), so no step re-reads a whole K
    cache to keep its scores current."""

    def __init__(self, e_low, e_high, zeta=None, keep=None, zeta_max: float = 0.0, tile_size: int = TILE_SIZE):
        self.e_low, self.e_high, self.zeta, self.keep = e_low, e_high, zeta, keep
        self.zeta_max = zeta_max
        self.tile_size = tile_size  # tokens per tile the scores were formed over

    def as_pair(self):
        return self.e_low, self.e_high

    @classmethod
    def allocate(cls, rows: int, max_tiles: int, device, zeta_max: float = 0.0,
                 tile_size: int = TILE_SIZE) -> "TileScores":
        """Zeroed (rows, max_tiles) score tensors to fill with `update`."""
        z = lambda dt: torch.zeros((rows, max_tiles), dtype=dt, device=device)
        return cls(z(torch.float32), z(torch.float32), z(torch.float32), z(torch.bool), zeta_max=zeta_max,
                   tile_size=tile_size)

    def update(self, keys: torch.Tensor, first_tile: int, count: int = 1, *, block_tables=None,
               context_lens=None, k_scale=None) -> "TileScores":
        """Rescore tiles [first_tile, first_tile + count) of every row in
        place.  `keys` is the (rows, S, d) K cache, or with `block_tables`
        the paged (num_blocks, Hkv, block_size, d) cache (rows = b*Hkv + h);
        `k_scale`: optional (rows, T) per-tile scales.  Tiles not wholly
        inside a row's length (context_lens) score as partial tails."""
        T = self.e_high.shape[1]
        if not 0 <= first_tile and first_tile + count <= T:
            raise ValueError(f"tiles [{first_tile}, {first_tile + count}) outside the cache's {T} tiles")
        if block_tables is not None:
            X.require_gpu(keys, block_tables)
            nb, hkv, bs, d = keys.shape
            ts = self.tile_size
            kv = X.paged_layout(keys, keys, block_tables, -(-(block_tables.shape[1] * bs) // ts), tile_size=ts)
        else:
            squeeze = keys.ndim == 2
            keys = keys.unsqueeze(0) if squeeze else keys
            X.require_gpu(keys)
            kv = X.rows_layout(keys, None, tile_size=self.tile_size)
        if first_tile + count > kv.num_tiles:
            raise ValueError(f"keys hold {kv.num_tiles} tiles, tiles up to {first_tile + count} requested")
        if kv.num_rows > self.e_high.shape[0]:
            raise ValueError(f"keys have {kv.num_rows} rows, the cache {self.e_high.shape[0]}")
        if context_lens is not None:
            kv.lengths = context_lens.to(device=keys.device, dtype=torch.int32).contiguous()
        if isinstance(k_scale, torch.Tensor):
            kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, kv.num_rows, kv.num_tiles,
                                                                     keys.device)
        X.score_tile_range(kv, first_tile, count, self.e_low, self.e_high, self.zeta,
                           None if self.keep is None else self.keep.view(torch.uint8), self.zeta_max)
        return self


def fwht_tiles(keys: torch.Tensor, *, tile_size: int = TILE_SIZE) -> torch.Tensor:
    """The full transform X = W_TS @ K_tile of every tile of (S, d) or
    (rows, S, d) keys, float32 (rows, T, TS, d) (or (T, TS, d)); TS = 64 or
    `tile_size`."""
    squeeze = keys.ndim == 2
    if squeeze:
        keys = keys.unsqueeze(0)
    X.require_gpu(keys)
    X.check_tile_size(tile_size)
    kv = X.rows_layout(keys, None, tile_size=tile_size)
    out = X.fwht_tiles(kv)
    return out[0] if squeeze else out


def print_kernel_metadata(match: str = "score_kernel"):
    """Print the compiled kernels' LDS use, registers, scratch and spills
    (fwht_fused_prototype.py:329-385).  The reference triggers Triton's JIT
    and reads its metadata for the FWHT kernel; here every kernel is built
    ahead of time, so the figures are read from the gfx950 code objects of
    liborthocache_hip.so (no launch, no GPU needed).  `match` selects kernels
    by a substring of their demangled names: the tile-scoring kernels by
    default, '' for all.  Returns the printed rows."""
    from ..kernel_metadata import print_kernel_metadata as _print
    return _print(match)
