"""Decode-attention kernels of OrthoCache for MI355X (gfx950).

The subpackage keeps the reference's module names (triton_kernels.*) so that
existing imports keep working; every kernel behind them is hand-written HIP
in liborthocache_hip.so.  The block-sparse and indirect attention entry
points run the decode kernel with a given tile mask.
"""

from .fwht_fused_prototype import (  # noqa: F401
    TILE_SIZE, BAND_DC_64, BAND_LOW_64, BAND_MID_64, BAND_HIGH_64,
    generate_walsh_matrix, triton_fwht_eviction, score_tiles, fwht_tiles, TileScores, print_kernel_metadata,
)
from .fused_eviction import fused_orthocache_attention, fused_orthocache_attention_v2  # noqa: F401
from .gqa_eviction import fused_orthocache_attention_v3_gqa  # noqa: F401
from .paged_eviction import fused_orthocache_attention_paged  # noqa: F401
from .sparse_attention import triton_block_sparse_attention  # noqa: F401
from .indirect_attention import triton_indirect_attention  # noqa: F401

__all__ = [
    "triton_block_sparse_attention",
    "triton_indirect_attention",
    "triton_fwht_eviction",
    "generate_walsh_matrix",
    "score_tiles",
    "fwht_tiles",
    "TileScores",
    "print_kernel_metadata",
    "fused_orthocache_attention",
    "fused_orthocache_attention_v2",
    "fused_orthocache_attention_v3_gqa",
    "fused_orthocache_attention_paged",
]
