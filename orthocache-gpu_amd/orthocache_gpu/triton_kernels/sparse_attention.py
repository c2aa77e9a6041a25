"""Block-sparse single-query attention (reference module
triton_kernels/sparse_attention.py): only the KV blocks whose block_mask
entry is True are read.

The HIP decode kernel runs it with a given tile mask (OC_GATE_MASK): a
block of block_size tokens is block_size / 64 of its 64-token tiles, so the
retained blocks are streamed with the same balanced, matrix-core decode as
the spectral gates, and no evicted block is read.
"""

from __future__ import annotations

import torch

from .. import _launch as X
from .fwht_fused_prototype import TILE_SIZE

BLOCK_SIZE: int = 512


def _tiles_per_block(block_size: int) -> int:
    if block_size % TILE_SIZE:
        raise NotImplementedError(f"block_size must be a multiple of {TILE_SIZE} tokens, got {block_size}")
    return block_size // TILE_SIZE


def triton_block_sparse_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                                  block_mask: torch.Tensor, block_size: int = BLOCK_SIZE) -> torch.Tensor:
    """q (1, head_dim); keys / values (num_blocks * block_size, head_dim);
    block_mask (num_blocks,) bool, True = attend.  Returns (1, head_dim) in
    q's dtype: softmax(q K^T / sqrt(d)) V over the retained blocks, float32
    accumulation, zeros when no block is retained (sparse_attention.py:208-279)."""
    assert q.ndim == 2 and q.shape[0] == 1, f"q must be (1, head_dim), got {q.shape}"
    num_tokens = keys.shape[0]
    num_blocks = num_tokens // block_size
    assert num_tokens == num_blocks * block_size, (
        f"keys length {num_tokens} not divisible by block_size {block_size}"
    )
    assert block_mask.shape == (num_blocks,), f"block_mask shape {block_mask.shape} != ({num_blocks},)"
    tpb = _tiles_per_block(block_size)
    device = X.require_gpu(q, keys, values)
    tile_mask = X.tile_mask_from_blocks(num_blocks, tpb, device, block_mask=block_mask)
    return X.masked_decode(q, keys, values, tile_mask)
