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

# the last few matrices validated, with their version counter and scale; the
# entries hold the tensors, so an address cannot be reused while cached
_WALSH_SCALE: list = []


def _walsh_scale(walsh_matrix: torch.Tensor, tile_size: int) -> float:
    """The band-norm kernel transforms with W64 = H64 / 8 (what
    generate_walsh_matrix(64) returns).  A caller's matrix c * H64 (the
    reference takes any matrix; its evaluation code passes the unnormalised
    H64, c = 1) gives norms 8c times the kernel's: the factor is returned,
    and any matrix that is not a scalar multiple of H64 is refused.  For c a
    power of two (1/8, 1, ...) the scaled norms are bit for bit those of
    W @ K; otherwise they carry one more rounding."""
    if tile_size != TILE_SIZE or tuple(walsh_matrix.shape) != (TILE_SIZE, TILE_SIZE):
        raise NotImplementedError(f"the HIP band-norm kernel implements {TILE_SIZE}-token tiles only")
    for m, version, scale in _WALSH_SCALE:
        if m is walsh_matrix and version == walsh_matrix._version:
            return scale
    w = walsh_matrix.float()
    c = float(w[0, 0])
    ref = generate_walsh_matrix(TILE_SIZE).to(w.device) * (8.0 * c)
    if c <= 0 or not torch.equal(w, ref):
        raise NotImplementedError("walsh_matrix must be a positive multiple of the 64-point Sylvester matrix "
                                  "(generate_walsh_matrix(64) or the unnormalised H64)")
    _WALSH_SCALE.insert(0, (walsh_matrix, walsh_matrix._version, 8.0 * c))
    del _WALSH_SCALE[8:]
    return 8.0 * c


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
        scale = _walsh_scale(walsh_matrix, k_tile.shape[0])
        if not 0 <= kv_head < self.num_kv_heads or not 0 <= tile_idx < self.max_tiles:
            raise IndexError(f"(kv_head {kv_head}, tile {tile_idx}) outside ({self.num_kv_heads}, {self.max_tiles})")
        kv = X.rows_layout(k_tile.unsqueeze(0), None)
        X.band_norms(kv, 0, 1, (high_start, high_end), self.cache[kv_head:kv_head + 1],
                     self.valid_tiles[kv_head:kv_head + 1], tile_offset=tile_idx)
        if scale != 1.0:
            self.cache[kv_head, tile_idx:tile_idx + 1].mul_(scale)
        self._populated = True

    def populate_from_keys(self, keys: torch.Tensor, walsh_matrix: torch.Tensor, tile_size: int = 64,
                           high_start: int = 48, high_end: int = 64):
        """All complete tiles of (num_kv_heads, seq_len, head_dim) keys in one
        launch (norm_cache.py:90-117)."""
        scale = _walsh_scale(walsh_matrix, tile_size)
        num_kv_heads, seq_len, _ = keys.shape
        heads = min(num_kv_heads, self.num_kv_heads)
        tiles = min(seq_len // tile_size, self.max_tiles)
        if heads and tiles:
            kv = X.rows_layout(keys[:heads, :tiles * tile_size], None)
            X.band_norms(kv, 0, tiles, (high_start, high_end), self.cache, self.valid_tiles)
            if scale != 1.0:
                self.cache[:heads, :tiles].mul_(scale)
            self._populated = True
        return self

    def update_tiles(self, keys: torch.Tensor, first_tile: int, num_tiles: int = 1, high_start: int = 48,
                     high_end: int = 64, context_lens: Optional[torch.Tensor] = None, norm_scale: float = 1.0):
        """Append path: rescore tiles [first_tile, first_tile + num_tiles) of
        every kv head of the (num_kv_heads, S, head_dim) K cache (e.g. the
        tile a decode step just completed).  With context_lens (one per kv
        head), tiles not yet complete are left untouched.  norm_scale
        multiplies the W64 norms (8 for the unnormalised H64)."""
        heads = min(keys.shape[0], self.num_kv_heads)
        if first_tile < 0 or first_tile + num_tiles > min(keys.shape[1] // TILE_SIZE, self.max_tiles):
            raise ValueError(f"tiles [{first_tile}, {first_tile + num_tiles}) outside the cache")
        kv = X.rows_layout(keys[:heads], None)
        if context_lens is not None:
            kv.lengths = context_lens.to(device=keys.device, dtype=torch.int32).contiguous()
        if norm_scale != 1.0 and context_lens is not None:
            raise NotImplementedError("norm_scale with context_lens")
        X.band_norms(kv, first_tile, num_tiles, (high_start, high_end), self.cache, self.valid_tiles)
        if norm_scale != 1.0:
            self.cache[:heads, first_tile:first_tile + num_tiles].mul_(norm_scale)
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
