"""Attention over the retained 512-token blocks (src/orthocache_gpu/
adaptive_attention.py of the reference).

The reference compacts the block list (stream_compact) and loops over the
active blocks with an online softmax per head; here the block mask becomes
a 64-token tile mask and the split-K decode kernel (oc_decode with
OC_GATE_MASK) attends exactly the retained tiles, never reading an evicted
block's K or V.  Every query of q attends every retained key (no causal
mask), as in the reference; the output is bfloat16, as there.
"""

from __future__ import annotations

import torch

from . import _launch as X
from . import _native as N

BS = 512  # the default block size (the block_size arguments below override it per call)
_Q_CHUNK = 64  # query rows per decode call (the kernel's group limit)


def stream_compact(block_mask: torch.Tensor) -> tuple:
    """(active-first stable permutation int64 (num_blocks,), num_active int)
    (adaptive_attention.py:29-43)."""
    idx, cnt = X.stream_compact(block_mask)
    return idx, int(cnt.item())


def orthocache_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_mask: torch.Tensor,
                         block_size: int = 512) -> tuple:
    """q (seq_q, num_heads, head_dim), k_cache / v_cache (seq_k, num_heads,
    head_dim), block_mask (num_blocks,) bool, True = keep.  Returns (output
    (seq_q, num_heads, head_dim) bfloat16, stats) (adaptive_attention.py:159-215)."""
    device = X.require_gpu(q, k_cache, v_cache)
    seq_k = k_cache.shape[0]
    nb = block_mask.shape[0]
    keep = block_mask.to(device=device, dtype=torch.bool)
    num_active = int(keep.sum().item())
    if num_active == 0:
        return torch.zeros_like(q), {'num_active': 0, 'eviction_rate': 1.0, 'path': 'zero'}
    if block_size % X.TILE_SIZE:
        raise NotImplementedError(f"block_size {block_size} is not a multiple of the 64-token tile")
    tiles = keep.to(torch.uint8).repeat_interleave(block_size // X.TILE_SIZE)
    out = attend_tiles(q, k_cache, v_cache, tiles, nb * block_size)
    return out, {
        'num_active': num_active,
        'num_blocks': seq_k // block_size,
        'eviction_rate': 1.0 - num_active / (seq_k // block_size),
        'path': 'masked_decode',
    }


def attend_tiles(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, tile_mask: torch.Tensor,
                 tokens: int) -> torch.Tensor:
    """Every query of q (seq_q, heads, d) over the first `tokens` keys of
    k_cache / v_cache (seq_k, heads, d), attending the 64-token tiles whose
    tile_mask byte (uint8 (tokens // 64,), shared by the heads) is set;
    bfloat16 (seq_q, heads, d)."""
    seq_q, nh, hd = q.shape
    if tokens > k_cache.shape[0] or tokens % X.TILE_SIZE:
        raise ValueError(f"{tokens} tokens: more than the cache holds or not whole tiles")
    kv = X.rows_layout(k_cache[:tokens].permute(1, 0, 2), v_cache[:tokens].permute(1, 0, 2))
    tm = tile_mask.reshape(1, -1).expand(nh, -1)
    out = torch.empty((seq_q, nh, hd), dtype=torch.bfloat16, device=q.device)
    for s0 in range(0, seq_q, _Q_CHUNK):
        qq = q[s0:s0 + _Q_CHUNK].permute(1, 0, 2).contiguous()  # (heads, g, d)
        g = qq.shape[1]
        res = X.decode(kv, qq.reshape(nh * g, hd), g, gate=N.OC_GATE_MASK, threshold=0.0, mode=N.OC_MODE_CACHED,
                       out_dtype=torch.bfloat16, tile_mask=tm)
        out[s0:s0 + g] = res.out.view(nh, g, hd).permute(1, 0, 2)
    return out


def orthocache_attention_batched(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                 block_mask: torch.Tensor, block_size: int = 512) -> tuple:
    """q (batch, seq_q, heads, d), k_cache / v_cache (batch, seq_k, heads, d),
    one block_mask (num_blocks,) shared by the batch.  Returns (bfloat16
    (batch, seq_q, heads, d), stats) (adaptive_attention.py:246-294)."""
    device = X.require_gpu(q, k_cache, v_cache)
    seq_k = k_cache.shape[1]
    nb = block_mask.shape[0]
    keep = block_mask.to(device=device, dtype=torch.bool)
    num_active = int(keep.sum().item())
    if num_active == 0:
        return torch.zeros_like(q), {'num_active': 0, 'eviction_rate': 1.0, 'path': 'zero'}
    if block_size % X.TILE_SIZE:
        raise NotImplementedError(f"block_size {block_size} is not a multiple of the 64-token tile")
    tiles = keep.to(torch.uint8).repeat_interleave(block_size // X.TILE_SIZE)
    out = torch.stack([attend_tiles(q[b], k_cache[b], v_cache[b], tiles, nb * block_size)
                       for b in range(q.shape[0])])
    return out, {
        'num_active': num_active,
        'num_blocks': seq_k // block_size,
        'eviction_rate': 1.0 - num_active / (seq_k // block_size),
        'batch_size': q.shape[0],
        'path': 'masked_decode',
    }
