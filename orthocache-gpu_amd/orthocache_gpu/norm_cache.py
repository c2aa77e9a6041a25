"""Spectral norm cache: one float32 ||(W64 K_t)[high band]||_F per (kv head,
tile), filled at prefill and read by the O(1) decode gate
(triton_kernels/decode_gate.py).

Same class, methods and defaults as the reference's
`orthocache_gpu.norm_cache` (norm_cache.py:21-167); the norms come from the
band-norm kernel (oc_band_norms), one launch per call, instead of a W @ K
matmul and a `.item()` per tile.  Added: `update_tiles`, the append path
that rescores only the tiles a decode step completed.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _launch as X
from .triton_kernels.fwht_fused_prototype import TILE_SIZE, generate_walsh_matrix

_WALSH_OK = {}


def _require_walsh(walsh_matrix: torch.Tensor, tile_size: int) -> None:
    """The kernels implement the 64-point Walsh matrix W64 = H64/8 (the one
    generate_walsh_matrix(64) returns); any other matrix is refused."""
    if tile_size != TILE_SIZE or tuple(walsh_matrix.shape) != (TILE_SIZE, TILE_SIZE):
        raise NotImplementedError(f"the HIP band-norm kernel implements {TILE_SIZE}-token tiles only")
    key = (walsh_matrix.data_ptr(), walsh_matrix._version, walsh_matrix.device)
    if key not in _WALSH_OK:
        ref = generate_walsh_matrix(TILE_SIZE).to(walsh_matrix.device)
        if not torch.equal(walsh_matrix.float(), ref):
            raise NotImplementedError("walsh_matrix must be generate_walsh_matrix(64)")
        _WALSH_OK[key] = True


class SpectralNormCache:
    """Precomputed K-tile high-band norms for the O(1) decode gate
    (norm_cache.py:21-145).  cache: (num_kv_heads, max_tiles) float32;
    valid_tiles: (num_kv_heads,) int32, one past the highest tile stored."""

    def __init__(self, num_kv_heads: int, max_tiles: int, device: torch.device):
        self.cache = torch.zeros(num_kv_heads, max_tiles, dtype=torch.float32, device=device)
        self.valid_tiles = torch.zeros(num_kv_heads, dtype=torch.int32, device=device)
        self.num_kv_heads = num_kv_heads
        self.max_tiles = max_tiles
        self.device = device
        self._populated = False

    def update_prefill(self, kv_head: int, tile_idx: int, k_tile: torch.Tensor, walsh_matrix: torch.Tensor,
                       high_start: int, high_end: int):
        """||(W @ k_tile)[high_start:high_end]||_F of one (tile_size, head_dim)
        tile into cache[kv_head, tile_idx] (0 below 1e-38), and valid_tiles
        raised to tile_idx + 1 (norm_cache.py:58-88)."""
        _require_walsh(walsh_matrix, k_tile.shape[0])
        if not 0 <= kv_head < self.num_kv_heads or not 0 <= tile_idx < self.max_tiles:
            raise IndexError(f"(kv_head {kv_head}, tile {tile_idx}) outside ({self.num_kv_heads}, {self.max_tiles})")
        kv = X.rows_layout(k_tile.unsqueeze(0), None)
        X.band_norms(kv, 0, 1, (high_start, high_end), self.cache[kv_head:kv_head + 1],
                     self.valid_tiles[kv_head:kv_head + 1], tile_offset=tile_idx)
        self._populated = True

    def populate_from_keys(self, keys: torch.Tensor, walsh_matrix: torch.Tensor, tile_size: int = 64,
                           high_start: int = 48, high_end: int = 64):
        """All complete tiles of (num_kv_heads, seq_len, head_dim) keys in one
        launch (norm_cache.py:90-117)."""
        _require_walsh(walsh_matrix, tile_size)
        num_kv_heads, seq_len, _ = keys.shape
        heads = min(num_kv_heads, self.num_kv_heads)
        tiles = min(seq_len // tile_size, self.max_tiles)
        if heads and tiles:
            kv = X.rows_layout(keys[:heads, :tiles * tile_size], None)
            X.band_norms(kv, 0, tiles, (high_start, high_end), self.cache, self.valid_tiles)
            self._populated = True
        return self

    def update_tiles(self, keys: torch.Tensor, first_tile: int, num_tiles: int = 1, high_start: int = 48,
                     high_end: int = 64, context_lens: Optional[torch.Tensor] = None):
        """Append path: rescore tiles [first_tile, first_tile + num_tiles) of
        every kv head of the (num_kv_heads, S, head_dim) K cache (e.g. the
        tile a decode step just completed).  With context_lens (one per kv
        head), tiles not yet complete are left untouched."""
        heads = min(keys.shape[0], self.num_kv_heads)
        if first_tile < 0 or first_tile + num_tiles > min(keys.shape[1] // TILE_SIZE, self.max_tiles):
            raise ValueError(f"tiles [{first_tile}, {first_tile + num_tiles}) outside the cache")
        kv = X.rows_layout(keys[:heads], None)
        if context_lens is not None:
            kv.lengths = context_lens.to(device=keys.device, dtype=torch.int32).contiguous()
        X.band_norms(kv, first_tile, num_tiles, (high_start, high_end), self.cache, self.valid_tiles)
        self._populated = True
        return self

    def get_norm(self, kv_head: int, tile_idx: int) -> float:
        """Cached ||K_high||_F of one tile (a host read)."""
        return self.cache[kv_head, tile_idx].item()

    def get_norms_batch(self, kv_head: int) -> torch.Tensor:
        """Cached norms of one kv head's stored tiles, (valid_tiles,)."""
        n = self.valid_tiles[kv_head].item()
        return self.cache[kv_head, :n]

    @property
    def is_populated(self) -> bool:
        return self._populated

    @property
    def memory_bytes(self) -> int:
        return self.cache.nelement() * self.cache.element_size()

    def summary(self) -> str:
        total_tiles = self.valid_tiles.sum().item()
        return (f"SpectralNormCache: {self.num_kv_heads} heads × {self.max_tiles} max_tiles, "
                f"{total_tiles} populated, {self.memory_bytes / 1024:.1f} KB")


def create_norm_cache_for_model(model_config, max_seq_len: int = 32768, tile_size: int = 64,
                                device: torch.device = torch.device("cpu")) -> SpectralNormCache:
    """A cache sized for a model config with num_key_value_heads
    (norm_cache.py:148-167)."""
    cache = SpectralNormCache(model_config.num_key_value_heads, max_seq_len // tile_size, device)
    print(f"  Created {cache.summary()}")
    return cache
