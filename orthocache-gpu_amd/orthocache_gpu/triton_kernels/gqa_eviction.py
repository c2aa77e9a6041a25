"""GQA decode with the Cauchy-Schwarz spectral gate on MI355X.

Drop-in for src/orthocache_gpu/triton_kernels/gqa_eviction.py of the
reference.  A tile of kv head h is evicted for all G query heads
h*G .. h*G+G-1 iff max_g ||q_g||_2 * ||X[32:64]||_F <= tau, with norms
below 1e-38 clamped to 0 (gqa_eviction.py:222-239).  One workgroup keeps
the online-softmax states of all G query heads in registers while it
streams a kv tile once (the reference re-reads and re-writes the partial
state in global memory for every query head and tile, gqa_eviction.py:430-451).

Extensions (keyword-only): `k_scale` / `v_scale` per-tile tensors, `mode`
and `score_cache` (cached scores, K and V read for retained tiles only),
`context_lens` (tokens per kv row), `sync`.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from .. import _launch as X
from .. import _native as N
from .fused_eviction import _mode_code, _tile_size_supported
from .fwht_fused_prototype import BAND_HIGH_64, BAND_LOW_64, TILE_SIZE, generate_walsh_matrix  # noqa: F401


def _auto_num_splits_gqa(num_tiles: int, device: torch.device) -> int:
    """Same rule as v2 (gqa_eviction.py:502-508)."""
    if device.type != "cuda":
        return 1
    return X.auto_num_splits(num_tiles, device)


def fused_orthocache_attention_v3_gqa(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    tau: float,
    num_query_groups: int,
    num_splits: Optional[int] = None,
    tile_size: int = TILE_SIZE,
    k_scale=1.0,
    *,
    v_scale: Optional[torch.Tensor] = None,
    mode: str = "single_pass",
    score_cache=None,
    context_lens: Optional[torch.Tensor] = None,
    sync: bool = True,
    out: Optional[torch.Tensor] = None,
    return_partials: bool = False,
) -> Tuple[torch.Tensor, Dict[str, Any]]:
    """q (Hkv*G, d), keys/values (Hkv, S, d) -> (out (Hkv*G, d) in q.dtype,
    metadata) (gqa_eviction.py:511-639).  Query heads [h*G, (h+1)*G) share
    kv head h."""
    num_kv_heads, seq_len, head_dim = keys.shape
    num_query_heads = q.shape[0]
    G = num_query_groups
    num_tiles = seq_len // tile_size
    assert (head_dim & (head_dim - 1)) == 0 and head_dim > 0, f"head_dim ({head_dim}) must be a power of 2"
    assert (tile_size & (tile_size - 1)) == 0 and tile_size > 0, f"tile_size ({tile_size}) must be a power of 2"
    assert num_query_heads == num_kv_heads * G, (
        f"num_query_heads ({num_query_heads}) != num_kv_heads ({num_kv_heads}) × G ({G})")
    assert seq_len == num_tiles * tile_size, f"seq_len {seq_len} not divisible by tile_size {tile_size}"
    if num_splits is not None:
        assert num_splits > 0, f"num_splits ({num_splits}) must be greater than 0"
    _tile_size_supported(tile_size)
    input_dtype = q.dtype
    device = X.require_gpu(q, keys, values)
    if num_splits is None:
        num_splits = _auto_num_splits_gqa(num_tiles, device)

    kv = X.rows_layout(keys, values, tile_size=tile_size)
    kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, num_kv_heads, num_tiles, device)
    kv.v_scale_mode, kv.v_scales = X.vscale_mode(v_scale, num_kv_heads, num_tiles, device)
    if context_lens is not None:
        kv.lengths = context_lens.to(device=device, dtype=torch.int32).contiguous()
        kv.rows_per_length = 1
        if kv.lengths.numel() != num_kv_heads:
            raise ValueError(f"context_lens must have one entry per kv head ({num_kv_heads})")
    mode_c, scores = _mode_code(mode, score_cache, tile_size)
    res = X.decode(kv, q, G, gate=N.OC_GATE_CS, threshold=tau, mode=mode_c, scores=scores,
                   num_splits=num_splits, out_dtype=input_dtype, want_keep=sync,
                   want_partials=return_partials, out=out)
    metadata: Dict[str, Any] = {
        "num_splits": num_splits,
        "num_tiles": num_tiles,
        "num_kv_heads": num_kv_heads,
        "num_query_heads": num_query_heads,
        "num_query_groups": G,
        "tile_assignment": "interleaved",
        "gate_type": "cauchy_schwarz",
    }
    if sync:
        torch.cuda.synchronize(device)
        if context_lens is None:
            total = num_tiles * num_kv_heads
        else:
            total = int(((kv.lengths.clamp(min=0, max=seq_len) + tile_size - 1) // tile_size).sum().item())
        metadata.update(X.counts_metadata(res.keep[:, :num_tiles], total))
        metadata["eviction_mask"] = res.keep[:, :num_tiles].bool()
    if return_partials:
        metadata["partials"] = res.partials
    return res.out, metadata
