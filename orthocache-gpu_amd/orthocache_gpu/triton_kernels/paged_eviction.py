"""Paged (block-table) gated split-K decode on MI355X.

Drop-in for src/orthocache_gpu/triton_kernels/paged_eviction.py of the
reference: `fused_orthocache_attention_paged` keeps its signature,
assertions and metadata.  Token t of sequence b lives in physical block
block_tables[b, t // block_size] of the (num_blocks, num_kv_heads,
block_size, head_dim) caches; the decode kernel resolves one block id per
4-token group of a tile (block_size >= 4), so a 64-token spectral tile may
span several pages.  An fp8-e4m3fn key cache with a scalar k_scale is
dequantised as the reference does (k_cache.to(q.dtype) * k_scale in q's
dtype, paged_eviction.py:354-357), inside the kernel.

Extensions (keyword-only, reference behaviour by default):
  num_query_groups  G query heads per cache head (GQA),
  tau               use the Cauchy-Schwarz gate with this threshold instead
                    of the zeta gate,
  context_lens      int32 (num_seqs,) tokens per sequence (partial tail tile
                    retained and masked),
  k_scale / v_scale per-(row, tile) float32 scale tensors, row = b*Hkv + h,
  mode / score_cache, sync.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from .. import _launch as X
from .. import _native as N
from .fused_eviction import _mode_code, _tile_size_supported
from .fwht_fused_prototype import BAND_HIGH_64, BAND_LOW_64, TILE_SIZE, generate_walsh_matrix  # noqa: F401


def _auto_num_splits(num_tiles: int, device: torch.device) -> int:
    """Same rule as v2 (paged_eviction.py:40-46)."""
    if device.type != "cuda":
        return 1
    return X.auto_num_splits(num_tiles, device)


def fused_orthocache_attention_paged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    zeta_max: float,
    num_splits: Optional[int] = None,
    tile_size: int = TILE_SIZE,
    k_scale=1.0,
    *,
    num_query_groups: int = 1,
    tau: Optional[float] = None,
    context_lens: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    mode: str = "single_pass",
    score_cache=None,
    sync: bool = True,
    out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Dict[str, Any]]:
    """q (B, H, d), caches (NB, H/G, bs, d), block_tables int32 (B, max_blocks)
    -> (out (B, H, d) in q.dtype, metadata) (paged_eviction.py:323-445)."""
    num_seqs, num_heads, head_dim = q.shape
    block_size = k_cache.shape[2]
    max_blocks_per_seq = block_tables.shape[1]
    num_tiles = (max_blocks_per_seq * block_size) // tile_size
    seq_len = num_tiles * tile_size
    assert (head_dim & (head_dim - 1)) == 0 and head_dim > 0, f"head_dim ({head_dim}) must be a power of 2"
    assert (tile_size & (tile_size - 1)) == 0 and tile_size > 0, f"tile_size ({tile_size}) must be a power of 2"
    assert (block_size & (block_size - 1)) == 0 and block_size > 0, f"block_size ({block_size}) must be a power of 2"
    assert (seq_len % tile_size) == 0, f"seq_len {seq_len} not divisible by tile_size {tile_size}"
    if num_splits is not None:
        assert num_splits > 0, f"num_splits ({num_splits}) must be positive"
    _tile_size_supported(tile_size)
    if block_size < 4:
        raise NotImplementedError(f"block_size {block_size} < 4 is not supported by the HIP kernels")
    G = int(num_query_groups)
    num_kv_heads = k_cache.shape[1]
    if num_kv_heads * G != num_heads:
        raise ValueError(f"q has {num_heads} heads but the cache has {num_kv_heads} kv heads x G={G}")
    input_dtype = q.dtype
    device = X.require_gpu(q, k_cache, v_cache, block_tables)
    if context_lens is not None:
        num_tiles = -(-(max_blocks_per_seq * block_size) // tile_size)
    if num_splits is None:
        num_splits = _auto_num_splits(num_tiles, device)

    rows = num_seqs * num_kv_heads
    # fp8 K with a scalar k_scale: the reference dequantises the pool,
    # k_cache.to(q.dtype) * k_scale, and scales nothing after
    # (paged_eviction.py:354-357).  With bf16 q, a cached decode on pages of
    # >= 16 tokens does that rounding in-kernel as it widens K
    # (OC_KSCALE_DEQUANT) and reads a bf16 V beside the fp8 K as it is: no
    # copy of either pool.  Other shapes (and V of another type) dequantise
    # the pool first (bf16 q holds every fp8 value, so an unscaled K is only
    # widened to V's type).
    in_kernel = None
    if k_cache.dtype == torch.float8_e4m3fn and not isinstance(k_scale, torch.Tensor):
        ks = float(k_scale)
        k_scale = 1.0
        if (q.dtype == torch.bfloat16 and block_size >= 16 and mode == "cached"
                and v_cache.dtype in (torch.float8_e4m3fn, torch.bfloat16)):
            in_kernel = ks
        elif q.dtype != torch.bfloat16 or ks != 1.0:
            k_cache = X.dequant_fp8(k_cache, ks, q.dtype)
    vmode, vscales = X.vscale_mode(v_scale, rows, num_tiles, device)
    lengths = None
    if context_lens is not None:
        if context_lens.numel() != num_seqs:
            raise ValueError(f"context_lens must have {num_seqs} entries")
        lengths = context_lens.to(device=device, dtype=torch.int32).clamp(
            min=0, max=max_blocks_per_seq * block_size).contiguous()
    error_flag = torch.zeros(1, dtype=torch.int32, device=device) if sync else None
    gate, thr = (N.OC_GATE_CS, tau) if tau is not None else (N.OC_GATE_ZETA, zeta_max)
    mode_c, scores = _mode_code(mode, score_cache, tile_size)
    q2 = q.reshape(num_seqs * num_heads, head_dim)
    out2 = None if out is None else out.view(num_seqs * num_heads, head_dim)

    def run(kc, dequant):
        kv = X.paged_layout(kc, v_cache, block_tables, num_tiles, keep_mixed=dequant is not None, tile_size=tile_size)
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, rows, num_tiles, device)
        if dequant is not None and dequant != 1.0:
            kv.k_scale_mode, kv.k_scale = N.OC_KSCALE_DEQUANT, dequant
        kv.v_scale_mode, kv.v_scales = vmode, vscales
        kv.lengths = lengths
        kv.error_flag = error_flag
        return kv, X.decode(kv, q2, G, gate=gate, threshold=thr, mode=mode_c, scores=scores,
                            num_splits=num_splits, out_dtype=input_dtype, want_keep=sync, out=out2)

    if in_kernel is None:
        kv, res = run(k_cache, None)
    else:
        try:
            kv, res = run(k_cache, in_kernel)
        except N.OrthoCacheHIPError as e:
            # a decode shape whose kernel neither dequantises K nor reads the
            # two types: the library refused before launching anything
            if e.code != N.OC_ERR_UNSUPPORTED:
                raise
            kv, res = run(X.dequant_fp8(k_cache, in_kernel, q.dtype) if in_kernel != 1.0 else k_cache, None)
    metadata: Dict[str, Any] = {
        "num_splits": num_splits,
        "num_tiles": num_tiles,
        "num_heads": num_heads,
        "num_seqs": num_seqs,
        "layout": "paged",
    }
    if sync:
        torch.cuda.synchronize(device)
        if int(kv.error_flag.item()) != 0:
            raise ValueError("block_tables holds a block id outside [0, num_blocks)")
        if context_lens is None:
            total = num_tiles * rows
        else:
            lens = kv.lengths.clamp(min=0, max=num_tiles * tile_size)
            total = int(((lens + tile_size - 1) // tile_size).sum().item()) * num_kv_heads
        metadata.update(X.counts_metadata(res.keep[:, :num_tiles], total))
    return res.out.view(num_seqs, num_heads, head_dim), metadata


def score_paged_tiles(k_cache: torch.Tensor, block_tables: torch.Tensor, tile_size: int = TILE_SIZE,
                      context_lens: Optional[torch.Tensor] = None, k_scale=None, q_dtype=None):
    """Cached scores of every tile of a paged key cache, rows = b*Hkv + h.

    Returns a TileScores whose e_low / e_high are (B*Hkv, T) float32; pass it
    as score_cache= with mode='cached'.  For an fp8 cache with a scalar
    k_scale, give q_dtype (the decode's query dtype) so that K is dequantised
    exactly as the decode does.
    """
    from .fwht_fused_prototype import TileScores
    _tile_size_supported(tile_size)
    X.require_gpu(k_cache, block_tables)
    nb, hkv, bs, d = k_cache.shape
    maxb = block_tables.shape[1]
    num_tiles = (maxb * bs) // tile_size if context_lens is None else -(-(maxb * bs) // tile_size)
    kv = X.paged_layout(k_cache, k_cache, block_tables, num_tiles, tile_size=tile_size)
    rows = block_tables.shape[0] * hkv
    if context_lens is not None:
        kv.lengths = context_lens.to(device=k_cache.device, dtype=torch.int32).clamp(
            min=0, max=maxb * bs).contiguous()
    if k_cache.dtype == torch.float8_e4m3fn and k_scale is not None and not isinstance(k_scale, torch.Tensor):
        # the decode's K: k_cache.to(q_dtype) * k_scale (paged_eviction.py:354-357)
        ks = float(k_scale)
        if q_dtype is None:
            raise ValueError("an fp8 cache with a scalar k_scale needs q_dtype (the decode's query dtype)")
        if q_dtype == torch.bfloat16:
            if ks != 1.0:
                kv.k_scale_mode, kv.k_scale = N.OC_KSCALE_DEQUANT, ks  # rounded to bf16 in the kernel
        else:
            kd = X.dequant_fp8(k_cache, ks, q_dtype)
            kv = X.paged_layout(kd, kd, block_tables, num_tiles, tile_size=tile_size)  # no V is read
            if context_lens is not None:
                kv.lengths = context_lens.to(device=k_cache.device, dtype=torch.int32).clamp(
                    min=0, max=maxb * bs).contiguous()
    if isinstance(k_scale, torch.Tensor):
        kv.k_scale_mode, kv.k_scale, kv.k_scales = X.kscale_mode(k_scale, rows, num_tiles, k_cache.device)
    e_low, e_high, zeta, keep = X.score_tiles(kv, 0.0)
    return TileScores(e_low[:, :num_tiles], e_high[:, :num_tiles], zeta[:, :num_tiles], tile_size=tile_size)
