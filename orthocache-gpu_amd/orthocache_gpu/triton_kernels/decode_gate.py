"""O(1) decode gate from cached K band norms (reference module
triton_kernels/decode_gate.py): each decode step reads one float per tile
from a SpectralNormCache instead of re-transforming K.

  compute_q_high_norm_exact  <- decode_gate.py:54-100   (oc_q_high_norms)
  decode_gate                <- decode_gate.py:188-245  (oc_decode_gate)
  apply_decode_mask[_vectorized] <- decode_gate.py:302-374 (oc_apply_tile_mask)

decode_gate follows the reference's GPU path (the Triton kernel): the
spatial ||q||_2, max over the G query heads of a kv head.  The keyword
q_norm="high" selects the Walsh-subspace ||q_high||_2 that the reference's
CPU path uses (_pytorch_decode_gate with tight=True, decode_gate.py:248-295).
Masks are True = evict.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _launch as X
from .._native import OC_QNORM_SPATIAL, OC_QNORM_WALSH_HIGH


def compute_q_high_norm_exact(q: torch.Tensor, low_band: int = 8) -> torch.Tensor:
    """||q_high||_2 over the last dimension: sqrt(max(||q||^2 - sum_i S_i^2
    / bs, 0)) with S_i the sums of the low_band blocks of bs = head_dim /
    low_band elements (the projection onto block-constant vectors).
    Returns q.shape[:-1] float32."""
    head_dim = q.shape[-1]
    assert head_dim % low_band == 0, f"head_dim ({head_dim}) must be divisible by low_band ({low_band})"
    return X.q_high_norms(q, low_band)


def decode_gate(q: torch.Tensor, norm_cache: torch.Tensor, tau: float, num_tiles: int, G: int,
                tile_size: int = 64, *, q_norm: str = "spatial",
                low_band: int = 8) -> Tuple[torch.Tensor, torch.Tensor]:
    """Eviction mask (num_kv_heads, max_tiles) bool (True = evict) and the
    per-kv-head q norms (num_kv_heads,) from q (num_q_heads, head_dim) and
    cached ||K_high||_F norm_cache (num_kv_heads, max_tiles): evict tile t of
    kv head h iff max_g ||q_g|| * norm_cache[h, t] <= tau * tile_size *
    head_dim, for t < num_tiles (decode_gate.py:188-245)."""
    if q_norm not in ("spatial", "high"):
        raise ValueError(f"q_norm must be 'spatial' or 'high', got {q_norm!r}")
    num_q_heads, head_dim = q.shape
    tau_norm = tau * float(tile_size * head_dim)
    mode = OC_QNORM_SPATIAL if q_norm == "spatial" else OC_QNORM_WALSH_HIGH
    return X.decode_gate(q, norm_cache, tau_norm, num_tiles, G, mode, low_band)


def apply_decode_mask(logits: torch.Tensor, mask: torch.Tensor, G: int, tile_size: int = 64,
                      num_tiles: Optional[int] = None) -> torch.Tensor:
    """logits (num_q_heads, 1, seq_len): -inf over every evicted tile of the
    query head's kv head, in place; returns logits (decode_gate.py:302-331)."""
    if num_tiles is None:
        num_tiles = logits.shape[2] // tile_size
    X.apply_tile_mask(logits, mask, G, tile_size, min(num_tiles, mask.shape[1]))
    return logits


def apply_decode_mask_vectorized(logits: torch.Tensor, mask: torch.Tensor, G: int, tile_size: int = 64,
                                 num_tiles: Optional[int] = None) -> torch.Tensor:
    """Same result as apply_decode_mask (decode_gate.py:334-374)."""
    return apply_decode_mask(logits, mask, G, tile_size, num_tiles)
