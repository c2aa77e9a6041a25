"""Indirect-indexing single-query attention (reference module
triton_kernels/indirect_attention.py): only the KV blocks listed in
active_indices are read, in place, with no compaction copy.

The index list becomes a tile mask on the device (oc_tile_mask_from_blocks)
and the HIP decode kernel attends exactly those tiles (OC_GATE_MASK).  A
block listed twice is attended once (the reference would weight it twice);
an index outside the cache raises ValueError (the reference reads out of
bounds).
"""

from __future__ import annotations

import torch

from .. import _launch as X
from .sparse_attention import BLOCK_SIZE, _tiles_per_block


def triton_indirect_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                              active_indices: torch.Tensor, num_active: int,
                              block_size: int = BLOCK_SIZE) -> torch.Tensor:
    """q (1, head_dim); keys / values (num_blocks * block_size, head_dim), the
    uncompacted cache; active_indices (>= num_active,) block indices.
    Returns (1, head_dim) in q's dtype (indirect_attention.py:200-286)."""
    assert q.ndim == 2 and q.shape[0] == 1, f"q must be (1, head_dim), got {q.shape}"
    assert active_indices.ndim == 1, f"active_indices must be 1-D, got shape {active_indices.shape}"
    assert num_active <= active_indices.shape[0], (
        f"num_active ({num_active}) > len(active_indices) ({active_indices.shape[0]})"
    )
    if num_active == 0:
        X.require_gpu(q)
        return torch.zeros_like(q)
    tpb = _tiles_per_block(block_size)
    device = X.require_gpu(q, keys, values)
    num_blocks = keys.shape[0] // block_size
    tile_mask = X.tile_mask_from_blocks(num_blocks, tpb, device, indices=active_indices[:num_active])
    # tokens past the last whole block are never attended
    keys = keys[:num_blocks * block_size]
    values = values[:num_blocks * block_size]
    return X.masked_decode(q, keys, values, tile_mask)
