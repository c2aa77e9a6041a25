"""Fused FWHT + zeta gate + split-K flash-decode on MI355X.

Drop-in for src/orthocache_gpu/triton_kernels/fused_eviction.py of the
reference: `fused_orthocache_attention` (v1, single head) and
`fused_orthocache_attention_v2` (multi-head split-K) keep their signatures,
assertion messages, tile assignment ({s + kP}, P from _auto_num_splits) and
metadata keys.  Both run liborthocache_hip's oc_decode (one decode kernel
plus the log-sum-exp merge); tensors must be on the GPU.

Extensions (keyword-only, reference behaviour by default):
  k_scale  a tensor of per-tile float32 scales (fp8 K) instead of a scalar,
  v_scale  per-tile float32 V scales,
  mode     'single_pass' (score every tile from K, read V of retained tiles)
           or 'cached' (read `score_cache` scores, read K and V of retained
           tiles only),
  sync     False skips the final torch.cuda.synchronize() and the counts.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from .. import _launch as X
from .. import _native as N
from .fwht_fused_prototype import BAND_HIGH_64, BAND_LOW_64, TILE_SIZE, generate_walsh_matrix  # noqa: F401


def _auto_num_splits(num_tiles: int, device: torch.device) -> int:
    """P = min(#CU, max(1, T // 4), T), at least 1 (fused_eviction.py:556-570)."""
    if device.type != "cuda":
        return 1
    return X.auto_num_splits(num_tiles, device)


def _check_common(head_dim: int, tile_size: int, seq_len: int, num_tiles: int) -> None:
    assert (head_dim & (head_dim - 1)) == 0 and head_dim > 0, f"head_dim ({head_dim}) must be a power of 2"
    assert (tile_size & (tile_size - 1)) == 0 and tile_size > 0, f"tile_size ({tile_size}) must be a power of 2"
    assert seq_len == num_tiles * tile_size, f"seq_len {seq_len} not divisible by tile_size {tile_size}"


def _tile_size_supported(tile_size: int) -> None:
    """Powers of two up to 256 tokens (the reference takes any power of two,
    fused_eviction.py:610; 64 runs the tuned kernels, the others the
    portable ones)."""
    X.check_tile_size(tile_size)


def _mode_code(mode: str, score_cache, tile_size: int = TILE_SIZE
               ) -> Tuple[int, Optional[Tuple[torch.Tensor, torch.Tensor]]]:
    if mode == "single_pass":
        return N.OC_MODE_SINGLE_PASS, None
    if mode == "cached":
        if score_cache is None:
            raise ValueError("mode='cached' needs score_cache= (see fwht_fused_prototype.score_tiles)")
        cache_ts = getattr(score_cache, "tile_size", tile_size)
        if cache_ts != tile_size:
            raise ValueError(f"score_cache holds scores of {cache_ts}-token tiles, the decode uses {tile_size}")
        pair = score_cache.as_pair() if hasattr(score_cache, "as_pair") else tuple(score_cache)
        return N.OC_MODE_CACHED, (pair[0].float(), pair[1].float())
    raise ValueError(f"mode must be 'single_pass' or 'cached', got {mode!r}")


def fused_orthocache_attention_v2(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    zeta_max: float,
    num_splits: Optional[int] = None,
    tile_size: int = TILE_SIZE,
    k_scale=1.0,
    *,
    v_scale: Optional[torch.Tensor] = None,
    mode: str = "single_pass",
    score_cache=None,
    sync: bool = True,
    out: Optional[torch.Tensor] = None,
    return_partials: bool = False,
) -> Tuple[torch.Tensor, Dict[str, Any]]:
    """Multi-head zeta-gated split-K decode (fused_eviction.py:573-691).

    q (H, d), keys/values (H, S, d) -> (out (H, d) in q.dtype, metadata).
    Tiles whose e_high/(e_low+1e-6) exceeds zeta_max are skipped; split s
    of each head owns tiles {s, s+P, s+2P, ...}.
    """
    num_heads = q.shape[0]
    head_dim = q.shape[-1]
    seq_len = keys.shape[1]
    num_tiles = seq_len // tile_size
    _check_common(head_dim, tile_size, seq_len, num_tiles)
    if num_splits is not None:
        assert num_splits > 0, f"num_splits ({num_splits}) must be greater than 0"
    _tile_size_supported(tile_size)
    input_dtype = q.dtype
    device = X.require_gpu(q, keys, values)
    if num_splits is None:
        num_splits = _auto_num_splits(num_tiles, device)

    kv = X.rows_layout(keys, values, tile_size=tile_size)
    kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, num_heads, num_tiles, device)
    kv.v_scale_mode, kv.v_scales = X.vscale_mode(v_scale, num_heads, num_tiles, device)
    mode_c, scores = _mode_code(mode, score_cache, tile_size)
    res = X.decode(kv, q, 1, gate=N.OC_GATE_ZETA, threshold=zeta_max, mode=mode_c, scores=scores,
                   num_splits=num_splits, out_dtype=input_dtype, want_keep=sync,
                   want_partials=return_partials, out=out)
    metadata: Dict[str, Any] = {
        "num_splits": num_splits,
        "num_tiles": num_tiles,
        "num_heads": num_heads,
        "tile_assignment": "interleaved",
    }
    if sync:
        torch.cuda.synchronize(device)
        metadata.update(X.counts_metadata(res.keep[:, :num_tiles], num_tiles * num_heads))
        metadata["eviction_mask"] = res.keep[:, :num_tiles].bool()
    if return_partials:
        metadata["partials"] = res.partials
    return res.out, metadata


def fused_orthocache_attention(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    zeta_max: float,
    tile_size: int = TILE_SIZE,
    return_mask: bool = False,
    k_scale=1.0,
    *,
    v_scale: Optional[torch.Tensor] = None,
    mode: str = "single_pass",
    score_cache=None,
    sync: bool = True,
) -> Tuple[torch.Tensor, Dict[str, Any]]:
    """Single-head zeta-gated decode (fused_eviction.py:698-800).

    q (1, d), keys/values (num_tiles*64, d) -> (out (1, d) in q.dtype,
    metadata with tiles_retained / tiles_evicted / eviction_rate and, when
    return_mask, eviction_mask (bool, True = retained)).
    """
    assert q.ndim == 2 and q.shape[0] == 1, f"q must be (1, head_dim), got {q.shape}"
    head_dim = q.shape[-1]
    num_tokens = keys.shape[0]
    num_tiles = num_tokens // tile_size
    assert (head_dim & (head_dim - 1)) == 0 and head_dim > 0, f"head_dim ({head_dim}) must be a power of 2"
    assert (tile_size & (tile_size - 1)) == 0 and tile_size > 0, f"tile_size ({tile_size}) must be a power of 2"
    assert num_tokens == num_tiles * tile_size, f"seq_len {num_tokens} not divisible by tile_size {tile_size}"
    _tile_size_supported(tile_size)
    input_dtype = q.dtype
    device = X.require_gpu(q, keys, values)

    kv = X.rows_layout(keys.unsqueeze(0), values.unsqueeze(0), tile_size=tile_size)
    kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, 1, num_tiles, device)
    kv.v_scale_mode, kv.v_scales = X.vscale_mode(v_scale, 1, num_tiles, device)
    mode_c, scores = _mode_code(mode, score_cache, tile_size)
    if scores is not None:
        scores = (scores[0].reshape(1, -1), scores[1].reshape(1, -1))
    res = X.decode(kv, q, 1, gate=N.OC_GATE_ZETA, threshold=zeta_max, mode=mode_c, scores=scores,
                   num_splits=X.auto_num_splits(num_tiles, device), out_dtype=input_dtype,
                   want_keep=sync or return_mask)
    metadata: Dict[str, Any] = {}
    if sync:
        torch.cuda.synchronize(device)
        metadata.update(X.counts_metadata(res.keep[:, :num_tiles], num_tiles))
    if return_mask:
        metadata["eviction_mask"] = res.keep[0, :num_tiles].bool()
    return res.out, metadata
