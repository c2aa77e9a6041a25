"""Host-side plumbing shared by the drop-in entry points: tensor checks,
KV descriptors, workspace reuse and the oc_decode / oc_score_tiles calls.

torch is used for device memory and the current stream only; every
computation on the path runs in liborthocache_hip.
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import _native as N

TILE_SIZE = 64
MAX_SPLITS = 8192

_DTYPE_CODES = {
    torch.float32: N.OC_F32,
    torch.float16: N.OC_F16,
    torch.bfloat16: N.OC_BF16,
    torch.float8_e4m3fn: N.OC_FP8_E4M3FN,
}


def dtype_code(dt: torch.dtype, what: str, allow_fp8: bool = True) -> int:
    code = _DTYPE_CODES.get(dt)
    if code is None or (code == N.OC_FP8_E4M3FN and not allow_fp8):
        raise TypeError(f"orthocache_gpu: unsupported {what} dtype {dt}")
    return code


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "orthocache_gpu runs on an AMD GPU only: got a tensor on "
                f"'{t.device}'. Move the inputs to the GPU (there is no CPU fallback).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"orthocache_gpu: tensors on different devices ({dev} vs {t.device})")
    return dev


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _aligned(t: torch.Tensor, nbytes: int) -> bool:
    return t.data_ptr() % nbytes == 0


def _kv_align(head_dim: int, es: int) -> int:
    """Byte alignment the kernels need of every K / V offset: the tuned
    kernels' per-lane vector width at head_dim 64 / 128, one element for the
    portable kernels (other head dims)."""
    if head_dim not in (64, 128):
        return es
    return min(16, (head_dim // 16) * es)


def tuned_shape(head_dim: int, tile_size: int) -> bool:
    """head_dim 64 or 128 with 64-token tiles: the tuned kernels' shapes
    (every other power-of-two shape runs the portable kernels)."""
    return tile_size == TILE_SIZE and head_dim in (64, 128)


def check_tile_size(tile_size: int) -> None:
    """The reference takes any power-of-two tile size (fused_eviction.py:610);
    the portable kernels take up to 256 tokens."""
    if tile_size > 256:
        raise NotImplementedError(f"tiles of at most 256 tokens are supported, got {tile_size}")


_WIDTH = {torch.float8_e4m3fn: 1, torch.float16: 2, torch.bfloat16: 2, torch.float32: 4}


def harmonize_kv(k: torch.Tensor, v: Optional[torch.Tensor]):
    """The kernels read K and V in one element type.  When they differ, the
    narrower one is converted exactly to the wider one on the GPU (fp8-e4m3fn
    values are exact in f16, bf16 and f32; f16 with bf16 go to f32), as the
    reference's own fp8 paths mix an fp8 K with a wider V (test_fp8.py:43-57)."""
    if v is None or v.dtype == k.dtype:
        return k, v
    wk, wv = _WIDTH.get(k.dtype, 4), _WIDTH.get(v.dtype, 4)
    if wk == wv:
        return k.to(torch.float32), v.to(torch.float32)
    return (k.to(v.dtype), v) if wk < wv else (k, v.to(k.dtype))


def last_dim_ready(t: torch.Tensor, head_dim: int) -> torch.Tensor:
    """Returns `t` if its last dimension is contiguous and every other stride
    and the base pointer keep the kernel's vector loads aligned; otherwise a
    contiguous copy (the reference wrappers always copy, fused_eviction.py:636-638)."""
    es = t.element_size()
    al = _kv_align(head_dim, es)
    ok = t.stride(-1) == 1 and _aligned(t, al)
    if ok:
        for s in t.stride()[:-1]:
            if (s * es) % al:
                ok = False
    return t if ok else t.contiguous()


# ---------------------------------------------------------------- descriptors

@dataclass
class KVLayout:
    """Everything oc_kv_desc carries, plus the tensors it points to."""
    k: torch.Tensor
    v: Optional[torch.Tensor]
    head_dim: int
    num_rows: int
    num_tiles: int
    k_row_stride: int = 0
    k_token_stride: int = 0
    v_row_stride: int = 0
    v_token_stride: int = 0
    paged: bool = False
    block_size: int = 0
    num_kv_heads: int = 0
    block_tables: Optional[torch.Tensor] = None
    num_blocks: int = 0
    k_block_stride: int = 0
    k_head_stride: int = 0
    v_block_stride: int = 0
    v_head_stride: int = 0
    lengths: Optional[torch.Tensor] = None
    rows_per_length: int = 1
    num_tokens: int = 0  # tokens of every row without lengths (0: num_tiles * tile_size)
    tile_size: int = TILE_SIZE
    k_scale_mode: int = N.OC_KSCALE_NONE
    k_scale: float = 1.0
    k_scales: Optional[torch.Tensor] = None
    v_scale_mode: int = N.OC_VSCALE_NONE
    v_scales: Optional[torch.Tensor] = None
    error_flag: Optional[torch.Tensor] = None

    def struct(self) -> N.OcKvDesc:
        d = N.OcKvDesc()
        d.k = _ptr(self.k)
        d.v = _ptr(self.v)
        d.dtype = dtype_code(self.k.dtype, "K")
        if self.v is not None and self.v.dtype != self.k.dtype:
            if not (self.k.dtype == torch.float8_e4m3fn and self.v.dtype == torch.bfloat16):
                raise TypeError(f"orthocache_gpu: K and V dtypes differ ({self.k.dtype} vs {self.v.dtype})")
            d.v_dtype = N.OC_BF16  # read as it is by the decodes that take it
        d.head_dim = self.head_dim
        d.num_rows = self.num_rows
        d.num_tiles = self.num_tiles
        d.k_row_stride, d.k_token_stride = self.k_row_stride, self.k_token_stride
        d.v_row_stride, d.v_token_stride = self.v_row_stride, self.v_token_stride
        d.paged = 1 if self.paged else 0
        d.block_size = self.block_size
        d.num_kv_heads = self.num_kv_heads
        d.rows_per_length = self.rows_per_length
        d.block_tables = _ptr(self.block_tables)
        d.bt_stride = 0 if self.block_tables is None else self.block_tables.stride(0)
        d.num_blocks = self.num_blocks
        d.k_block_stride, d.k_head_stride = self.k_block_stride, self.k_head_stride
        d.v_block_stride, d.v_head_stride = self.v_block_stride, self.v_head_stride
        d.lengths = _ptr(self.lengths)
        d.num_tokens = self.num_tokens
        d.k_scale_mode = self.k_scale_mode
        d.k_scale = float(self.k_scale)
        d.k_scales = _ptr(self.k_scales)
        d.k_scales_row_stride = 0 if self.k_scales is None else self.k_scales.stride(0)
        d.v_scale_mode = self.v_scale_mode
        d.v_scales = _ptr(self.v_scales)
        d.v_scales_row_stride = 0 if self.v_scales is None else self.v_scales.stride(0)
        d.error_flag = _ptr(self.error_flag)
        d.tile_size = 0 if self.tile_size == TILE_SIZE else self.tile_size
        return d


def rows_layout(keys: torch.Tensor, values: Optional[torch.Tensor], partial_tail: bool = False,
                tile_size: int = TILE_SIZE) -> KVLayout:
    """(rows, S, d) K/V views (last dimension contiguous, any other strides).
    The tiles are the S // tile_size complete ones; with partial_tail a last
    partial tile is included (as the descriptor's num_tokens = S, one length
    for every row)."""
    rows, s_len, d = keys.shape
    if values is not None and values.shape != keys.shape:
        raise ValueError(f"keys {tuple(keys.shape)} and values {tuple(values.shape)} must have the same shape")
    keys, values = harmonize_kv(keys, values)
    keys = last_dim_ready(keys, d)
    if values is not None:
        values = last_dim_ready(values, d)
    kv = KVLayout(
        k=keys, v=values, head_dim=d, num_rows=rows, num_tiles=s_len // tile_size,
        k_row_stride=keys.stride(0), k_token_stride=keys.stride(1),
        v_row_stride=0 if values is None else values.stride(0),
        v_token_stride=0 if values is None else values.stride(1), tile_size=tile_size)
    if partial_tail and s_len % tile_size:
        kv.num_tiles += 1
        kv.num_tokens = s_len
    return kv


def mixed_fp8k_bf16v(k: torch.Tensor, v: Optional[torch.Tensor]) -> bool:
    """fp8 K beside bf16 V, which the per-wave-prologue decode reads as they are."""
    return v is not None and k.dtype == torch.float8_e4m3fn and v.dtype == torch.bfloat16


def paged_layout(k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                 num_tiles: int, *, keep_mixed: bool = False, tile_size: int = TILE_SIZE) -> KVLayout:
    """(num_blocks, num_kv_heads, block_size, d) caches + int32 block table.
    keep_mixed: an fp8 K beside a bf16 V is passed as it is (no conversion);
    decodes that cannot read it fail with OC_ERR_UNSUPPORTED."""
    nb, hkv, bs, d = k_cache.shape
    if v_cache.shape != k_cache.shape:
        raise ValueError(f"k_cache {tuple(k_cache.shape)} and v_cache {tuple(v_cache.shape)} must have the same shape")
    if block_tables.dim() != 2:
        raise ValueError("block_tables must be 2-D (num_seqs, max_blocks)")
    if not (keep_mixed and mixed_fp8k_bf16v(k_cache, v_cache)):
        k_cache, v_cache = harmonize_kv(k_cache, v_cache)
    k_cache = last_dim_ready(k_cache, d)
    v_cache = last_dim_ready(v_cache, d)
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(-1) != 1:
        block_tables = block_tables.contiguous()
    return KVLayout(
        k=k_cache, v=v_cache, head_dim=d, num_rows=block_tables.shape[0] * hkv, num_tiles=num_tiles,
        k_token_stride=k_cache.stride(2), v_token_stride=v_cache.stride(2),
        paged=True, block_size=bs, num_kv_heads=hkv, block_tables=block_tables, num_blocks=nb,
        k_block_stride=k_cache.stride(0), k_head_stride=k_cache.stride(1),
        v_block_stride=v_cache.stride(0), v_head_stride=v_cache.stride(1),
        rows_per_length=hkv, tile_size=tile_size)


# ---------------------------------------------------------------- workspace

_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A reusable device buffer per (device, stream); calls on one stream are
    ordered, so they can share it.  It is allocated zeroed: oc_decode keeps
    its merge counters at the start of the workspace, needs them zero before
    the first call and leaves them zero."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream(device: torch.device) -> int:
    """The handle of torch's current stream on device (the raw query skips
    building a Stream object: about 0.3 against 1.9 us per call)."""
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------- split count

_CU_COUNT: Dict[int, int] = {}


def cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _CU_COUNT.get(idx)
    if n is None:
        n = torch.cuda.get_device_properties(idx).multi_processor_count
        _CU_COUNT[idx] = n
    return n


def auto_num_splits(num_tiles: int, device: torch.device) -> int:
    """P = max(1, min(#CU, max(1, T // 4), T)) (fused_eviction.py:556-570)."""
    return max(1, min(cu_count(device), max(1, num_tiles // 4), num_tiles))


# ---------------------------------------------------------------- calls

@dataclass
class DecodeResult:
    out: torch.Tensor
    keep: Optional[torch.Tensor] = None          # (rows, T) uint8
    split_counts: Optional[torch.Tensor] = None  # (rows, P) int32
    num_splits: int = 1
    partials: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None


def decode(kv: KVLayout, q: torch.Tensor, G: int, *, gate: int, threshold: float, mode: int = N.OC_MODE_SINGLE_PASS,
           scores: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, num_splits: Optional[int] = None,
           out_dtype: torch.dtype, want_keep: bool = False, want_partials: bool = False,
           out: Optional[torch.Tensor] = None, splits_per_group: Optional[int] = None,
           tile_mask: Optional[torch.Tensor] = None, portable: int = 0) -> DecodeResult:
    """One oc_decode call.  q is (rows*G, d) with a contiguous last dimension.
    With want_partials the per-split partial states (one workgroup per
    logical split) are returned as (m, l, acc) of shapes (rows*G, P) and
    (rows*G, P, d).  portable = 1 runs the portable kernels whatever the
    shape (they take every shape; the tuned ones run where they apply)."""
    device = require_gpu(q, kv.k, kv.v)
    d = kv.head_dim
    if q.stride(-1) != 1:
        q = q.contiguous()
    P = num_splits if num_splits is not None else auto_num_splits(kv.num_tiles, device)
    if not 1 <= P <= MAX_SPLITS:
        raise ValueError(f"num_splits {P} outside 1..{MAX_SPLITS}")
    rows_q = kv.num_rows * G
    if q.dim() != 2 or q.shape[0] != rows_q or q.shape[1] != d:
        raise ValueError(f"q must be ({rows_q}, {d}) for {kv.num_rows} kv rows x G={G}, got {tuple(q.shape)}")
    if out is None:
        out = torch.empty((rows_q, d), dtype=out_dtype, device=device)
    elif out.shape != (rows_q, d) or out.stride(-1) != 1 or out.device != device:
        raise ValueError(f"out must be a ({rows_q}, {d}) tensor on {device} with a contiguous last dim")
    keep = None
    if want_keep:
        keep = torch.zeros((kv.num_rows, max(kv.num_tiles, 1)), dtype=torch.uint8, device=device)
    p = N.OcDecodeParams()
    p.kv = kv.struct()
    p.q = q.data_ptr()
    p.q_dtype = dtype_code(q.dtype, "q", allow_fp8=False)
    p.G = G
    p.q_row_stride = q.stride(0)
    p.gate = gate
    p.mode = mode
    p.threshold = float(threshold)
    if scores is not None:
        e_low, e_high = scores
        for e in (e_low, e_high):
            if (e.dtype != torch.float32 or e.dim() != 2 or e.shape[0] < kv.num_rows or e.shape[1] < kv.num_tiles
                    or e.stride(1) != 1 or e.device != device or e.stride(0) != e_high.stride(0)):
                raise ValueError(f"score_cache must hold float32 ({kv.num_rows}, >= {kv.num_tiles}) tensors on "
                                 f"{device} with equal row strides")
        p.score_e_low = _ptr(e_low)
        p.score_e_high = _ptr(e_high)
        p.score_row_stride = e_high.stride(0)
    p.num_splits = P
    p.splits_per_group = 1 if want_partials else (splits_per_group or 0)
    p.portable = portable
    p.out_dtype = dtype_code(out.dtype, "out", allow_fp8=False)
    p.out = out.data_ptr()
    p.out_row_stride = out.stride(0)
    p.keep_out = _ptr(keep)
    p.keep_row_stride = 0 if keep is None else keep.stride(0)
    if tile_mask is not None:
        if (tile_mask.dtype != torch.uint8 or tile_mask.dim() != 2 or tile_mask.shape[0] < kv.num_rows
                or tile_mask.stride(1) != 1 or tile_mask.device != device):
            raise ValueError(f"tile_mask must be a uint8 ({kv.num_rows}, tiles) tensor on {device}")
        p.tile_mask, p.tile_mask_row_stride = tile_mask.data_ptr(), tile_mask.stride(0)
    partials = None
    if want_partials:
        pm = torch.empty((rows_q, P), dtype=torch.float32, device=device)
        pl = torch.empty((rows_q, P), dtype=torch.float32, device=device)
        pacc = torch.empty((rows_q, P, d), dtype=torch.float32, device=device)
        p.partial_m, p.partial_l, p.partial_acc = pm.data_ptr(), pl.data_ptr(), pacc.data_ptr()
        partials = (pm, pl, pacc)
    if kv.lengths is not None and kv.lengths.numel() * kv.rows_per_length < kv.num_rows:
        raise ValueError("lengths has fewer entries than the kv rows need")
    stream = current_stream(device)
    lib = N.lib()
    need = lib.oc_decode_workspace_size(ctypes.byref(p))
    if need:
        ws = workspace(device, stream, need)
        p.workspace = ws.data_ptr()
        p.workspace_bytes = ws.numel()
    with torch.cuda.device(device):
        N.check("oc_decode", lib.oc_decode(ctypes.byref(p), ctypes.c_void_p(stream)))
    return DecodeResult(out=out, keep=keep, num_splits=P, partials=partials)


def score_tiles(kv: KVLayout, zeta_max: float = 0.0, *, want_zeta: bool = True, want_keep: bool = True):
    """oc_score_tiles: returns (e_low, e_high, zeta|None, keep|None), each (rows, T)."""
    device = require_gpu(kv.k)
    shape = (kv.num_rows, max(kv.num_tiles, 1))
    e_low = torch.empty(shape, dtype=torch.float32, device=device)
    e_high = torch.empty(shape, dtype=torch.float32, device=device)
    zeta = torch.empty(shape, dtype=torch.float32, device=device) if want_zeta else None
    keep = torch.empty(shape, dtype=torch.uint8, device=device) if want_keep else None
    desc = kv.struct()
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_score_tiles", N.lib().oc_score_tiles(
            ctypes.byref(desc), float(zeta_max), e_low.data_ptr(), e_high.data_ptr(), _ptr(zeta),
            _ptr(keep), e_low.stride(0), ctypes.c_void_p(stream)))
    return e_low, e_high, zeta, keep


def score_tile_range(kv: KVLayout, first_tile: int, count: int, e_low: torch.Tensor, e_high: torch.Tensor,
                     zeta: Optional[torch.Tensor] = None, keep: Optional[torch.Tensor] = None,
                     zeta_max: float = 0.0) -> None:
    """oc_score_tile_range: rescore tiles [first_tile, first_tile + count) of
    every row into columns of existing (rows, >= T) score tensors."""
    device = require_gpu(kv.k, e_low, e_high)
    for t in (e_low, e_high, zeta, keep):
        if t is not None and (t.dim() != 2 or t.shape[0] < kv.num_rows or t.shape[1] < first_tile + count
                              or t.stride(1) != 1 or t.stride(0) != e_high.stride(0) or t.device != device):
            raise ValueError(f"score tensors must be ({kv.num_rows}, >= {first_tile + count}) with equal row "
                             f"strides on {device}")
    desc = kv.struct()
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_score_tile_range", N.lib().oc_score_tile_range(
            ctypes.byref(desc), int(first_tile), int(count), float(zeta_max), e_low.data_ptr(), e_high.data_ptr(),
            _ptr(zeta), _ptr(keep), e_high.stride(0), ctypes.c_void_p(stream)))


def band_norms(kv: KVLayout, first_tile: int, count: int, band: Tuple[int, int], out: torch.Tensor,
               valid_tiles: Optional[torch.Tensor] = None, tile_offset: int = 0) -> None:
    """oc_band_norms: ||(W64 K_t)[band]||_F of tiles [first_tile, first_tile +
    count) of every row into out (rows, >= T) float32.  With tile_offset
    > 0 the layout's tile 0 is numbered tile_offset (the descriptor's rows
    start tile_offset tiles before kv.k, which is never read): a single
    tile scored into column tile_offset of the outputs."""
    device = require_gpu(kv.k, out)
    if out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1 or out.shape[0] < kv.num_rows \
            or out.shape[1] < tile_offset + first_tile + count:
        raise ValueError(f"out must be float32 ({kv.num_rows}, >= {first_tile + count}) with contiguous rows")
    if valid_tiles is not None and (valid_tiles.dtype != torch.int32 or valid_tiles.numel() < kv.num_rows
                                    or not valid_tiles.is_contiguous()):
        raise ValueError("valid_tiles must be a contiguous int32 tensor with one entry per row")
    desc = kv.struct()
    if tile_offset:
        if kv.paged:
            raise ValueError("tile_offset applies to contiguous rows only")
        desc.k -= tile_offset * TILE_SIZE * kv.k_token_stride * kv.k.element_size()
        desc.num_tiles += tile_offset
        first_tile += tile_offset
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_band_norms", N.lib().oc_band_norms(
            ctypes.byref(desc), int(first_tile), int(count), int(band[0]), int(band[1]), out.data_ptr(),
            out.stride(0), _ptr(valid_tiles), ctypes.c_void_p(stream)))


def fwht_tiles(kv: KVLayout) -> torch.Tensor:
    """oc_fwht_tiles: (rows, T, TS, d) float32 spectra X = W_TS @ K_tile."""
    device = require_gpu(kv.k)
    out = torch.empty((kv.num_rows, kv.num_tiles, kv.tile_size, kv.head_dim), dtype=torch.float32, device=device)
    desc = kv.struct()
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_fwht_tiles", N.lib().oc_fwht_tiles(ctypes.byref(desc), out.data_ptr(),
                                                       ctypes.c_void_p(stream)))
    return out


def lse_merge(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    """oc_lse_merge of (rows, P) / (rows, P, d) float32 partials."""
    device = require_gpu(m, l, acc)
    rows, P = m.shape
    d = acc.shape[-1]
    m, l, acc = m.contiguous(), l.contiguous(), acc.contiguous()
    out = torch.empty((rows, d), dtype=out_dtype, device=device)
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_lse_merge", N.lib().oc_lse_merge(
            m.data_ptr(), l.data_ptr(), acc.data_ptr(), rows, P, d, out.data_ptr(),
            dtype_code(out_dtype, "out", allow_fp8=False), out.stride(0), ctypes.c_void_p(stream)))
    return out


def dequant_fp8(src: torch.Tensor, scale: float, out_dtype: torch.dtype) -> torch.Tensor:
    """oc_dequant_fp8: round_out(float(src) * scale) as a new out_dtype tensor."""
    device = require_gpu(src)
    src = src.contiguous()
    out = torch.empty(src.shape, dtype=out_dtype, device=device)
    n = src.numel()
    if n % 16:
        raise ValueError("fp8 tensor size must be a multiple of 16 elements")
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_dequant_fp8", N.lib().oc_dequant_fp8(
            src.data_ptr(), n, float(scale), dtype_code(out_dtype, "out", allow_fp8=False), out.data_ptr(),
            ctypes.c_void_p(stream)))
    return out


# the parameter blocks of hook_decode, per thread (a block's pointers are
# rewritten on every call, so two threads must not share one)
_HOOK_TLS = threading.local()


def hook_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, k_norms: torch.Tensor, G: int,
                tau_norm: float, low_band: int, want_stats: bool = True,
                stats_out: Optional[torch.Tensor] = None):
    """oc_hook_decode: the model hook's decode step in one call.  query
    (B, Hq, 1, d), key / value (B, Hkv, S, d) with a contiguous last
    dimension, k_norms float32 (>= Hkv, >= S // 64) with contiguous rows
    (shared by the batch).  Returns (out (B, Hq, 1, d) in query's dtype,
    gate statistics float32 (B * Hkv, 3) or None).  The parameter block is
    kept per shape and only its pointers and sizes are refreshed, so that
    a decode step costs one library call on the host."""
    B, Hq, _, d = query.shape
    Hkv, S = key.shape[1], key.shape[2]
    dt = query.dtype
    if key.dtype != dt or value.dtype != dt:
        # the reference decodes from query.float(), key.float(), value.float()
        # (perplexity_eval.py:590-592): with mixed types every operand is
        # widened to float32 (exact for float16 / bfloat16), the decode runs in
        # float32, and the output is rounded once to the query's type
        out, stats = hook_decode(query.float(), key.float(), value.float(), k_norms, G, tau_norm, low_band,
                                 want_stats, stats_out)
        return out.to(dt), stats
    rows = []
    for t in (key, value):
        if t.stride(3) != 1 or (B > 1 and t.stride(0) != Hkv * t.stride(1)):
            t = t.contiguous()
        rows.append(t)
    key, value = rows
    if query.stride(3) != 1 or (B > 1 and query.stride(0) != Hq * query.stride(1)):
        query = query.contiguous()
    device = query.device
    if not (device.type == "cuda" and key.device == device and value.device == device and k_norms.device == device):
        require_gpu(query, key, value, k_norms)  # raises with the reason
    if k_norms.dtype != torch.float32 or k_norms.stride(-1) != 1:
        raise ValueError("k_norms must be float32 with contiguous rows")
    skey = (device.index, dt, B, Hq, Hkv, d, key.stride(1), key.stride(2), value.stride(1), value.stride(2),
            query.stride(1), k_norms.stride(0), low_band)
    cache = getattr(_HOOK_TLS, "params", None)
    if cache is None:
        cache = _HOOK_TLS.params = {}
    p = cache.get(skey)
    if p is None:
        p = N.OcHookDecodeParams()
        p.q_row_stride = query.stride(1)
        p.k_row_stride, p.k_token_stride = key.stride(1), key.stride(2)
        p.v_row_stride, p.v_token_stride = value.stride(1), value.stride(2)
        p.dtype = dtype_code(dt, "q", allow_fp8=False)
        p.batch, p.num_kv_heads, p.G, p.head_dim = B, Hkv, G, d
        p.k_norms_stride = k_norms.stride(0)
        p.low_band = low_band
        p.num_splits = 0
        p.out_row_stride = d
        cache[skey] = p
    p.G = G
    p.kv_len = S
    p.tau_norm = tau_norm
    p.q, p.k, p.v, p.k_norms = query.data_ptr(), key.data_ptr(), value.data_ptr(), k_norms.data_ptr()
    out = torch.empty((B, Hq, 1, d), dtype=dt, device=device)
    if stats_out is not None:  # the caller's contiguous float32 (B * Hkv, 3) values, any view of them
        stats = stats_out
    else:
        stats = torch.empty((B * Hkv, 3), dtype=torch.float32, device=device) if want_stats else None
    p.out = out.data_ptr()
    p.gate_stats = None if stats is None else stats.data_ptr()
    lib = N.lib()
    stream = current_stream(device)
    ws = workspace(device, stream, lib.oc_hook_decode_workspace_size(ctypes.byref(p)))
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    if device.index == torch.cuda.current_device():
        rc = lib.oc_hook_decode(ctypes.byref(p), ctypes.c_void_p(stream))
    else:
        with torch.cuda.device(device):
            rc = lib.oc_hook_decode(ctypes.byref(p), ctypes.c_void_p(stream))
    if rc:
        N.check("oc_hook_decode", rc)
    return out, stats


def decode_gate(q: torch.Tensor, norm_cache: torch.Tensor, tau_norm: float, num_tiles: int, G: int,
                q_norm_mode: int, low_band: int = 8) -> Tuple[torch.Tensor, torch.Tensor]:
    """oc_decode_gate: (mask (Hkv, max_tiles) bool, True = evict; q_norms (Hkv,))."""
    device = require_gpu(q, norm_cache)
    if q.dim() != 2 or q.shape[0] % G:
        raise ValueError(f"q must be (num_kv_heads * G, head_dim), got {tuple(q.shape)} for G={G}")
    if q.stride(-1) != 1:
        q = q.contiguous()
    hkv = q.shape[0] // G
    if norm_cache.dtype != torch.float32:
        norm_cache = norm_cache.float()
    if norm_cache.dim() != 2 or norm_cache.shape[0] < hkv or norm_cache.stride(1) != 1:
        raise ValueError(f"norm_cache must be ({hkv}, max_tiles) float32 with contiguous rows")
    max_tiles = norm_cache.shape[1]
    if not 0 <= num_tiles <= max_tiles:
        raise ValueError(f"num_tiles {num_tiles} outside 0..{max_tiles}")
    mask = torch.empty((hkv, max_tiles), dtype=torch.bool, device=device)
    q_norms = torch.empty((hkv,), dtype=torch.float32, device=device)
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_decode_gate", N.lib().oc_decode_gate(
            q.data_ptr(), dtype_code(q.dtype, "q", allow_fp8=False), q.stride(0), hkv, G, q.shape[1],
            norm_cache.data_ptr(), norm_cache.stride(0), int(num_tiles), max_tiles, float(tau_norm), q_norm_mode,
            int(low_band), mask.data_ptr(), mask.stride(0), q_norms.data_ptr(), ctypes.c_void_p(stream)))
    return mask, q_norms


def q_high_norms(q: torch.Tensor, low_band: int) -> torch.Tensor:
    """oc_q_high_norms over the last dimension of q; returns q.shape[:-1] float32."""
    device = require_gpu(q)
    d = q.shape[-1]
    q2 = q.reshape(-1, d)
    if q2.stride(-1) != 1:
        q2 = q2.contiguous()
    out = torch.empty((q2.shape[0],), dtype=torch.float32, device=device)
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_q_high_norms", N.lib().oc_q_high_norms(
            q2.data_ptr(), dtype_code(q2.dtype, "q", allow_fp8=False), q2.shape[0], d, q2.stride(0), int(low_band),
            out.data_ptr(), ctypes.c_void_p(stream)))
    return out.view(q.shape[:-1])


def apply_tile_mask(logits: torch.Tensor, mask: torch.Tensor, G: int, tile_size: int, num_tiles: int) -> None:
    """oc_apply_tile_mask on (num_q_heads, 1, seq_len) or (num_q_heads, seq_len) logits, in place."""
    device = require_gpu(logits, mask)
    if logits.dim() == 3:
        if logits.shape[1] != 1:
            raise ValueError(f"logits must be (num_q_heads, 1, seq_len), got {tuple(logits.shape)}")
        rows = logits[:, 0, :]
    else:
        rows = logits
    if rows.stride(-1) != 1:
        raise ValueError("logits must be contiguous along the sequence")
    if mask.dtype not in (torch.bool, torch.uint8) or mask.dim() != 2 or mask.stride(1) != 1:
        raise ValueError("mask must be a (num_kv_heads, max_tiles) bool tensor with contiguous rows")
    if rows.shape[0] > mask.shape[0] * G or num_tiles > mask.shape[1]:
        raise ValueError("mask does not cover the logits' heads or tiles")
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_apply_tile_mask", N.lib().oc_apply_tile_mask(
            rows.data_ptr(), dtype_code(rows.dtype, "logits", allow_fp8=False), rows.shape[0], rows.shape[1],
            rows.stride(0), mask.data_ptr(), mask.stride(0), G, int(tile_size), int(num_tiles),
            ctypes.c_void_p(stream)))


def tile_mask_from_blocks(num_blocks: int, tiles_per_block: int, device, *, block_mask=None,
                          indices=None) -> torch.Tensor:
    """oc_tile_mask_from_blocks: (1, num_blocks * tiles_per_block) uint8 tile
    mask of a bool block mask or of an int32 block-index list (indices outside
    [0, num_blocks) raise ValueError after a device sync)."""
    tile_mask = torch.empty((1, max(1, num_blocks * tiles_per_block)), dtype=torch.uint8, device=device)
    err = None
    bm = ix = None
    count = 0
    if block_mask is not None:
        bm = block_mask.to(device=device, dtype=torch.uint8).contiguous()
    else:
        ix = indices.to(device=device, dtype=torch.int32).contiguous()
        count = ix.numel()
        err = torch.zeros(1, dtype=torch.int32, device=device)
    stream = current_stream(device)
    with torch.cuda.device(device):
        N.check("oc_tile_mask_from_blocks", N.lib().oc_tile_mask_from_blocks(
            _ptr(bm), _ptr(ix), count, num_blocks, tiles_per_block, tile_mask.data_ptr(), _ptr(err),
            ctypes.c_void_p(stream)))
    if err is not None and int(err.item()):
        raise ValueError(f"active_indices holds a block index outside [0, {num_blocks})")
    return tile_mask


def masked_decode(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, tile_mask: torch.Tensor) -> torch.Tensor:
    """One query row over (S, d) keys/values attending exactly the tiles whose
    tile_mask byte is set (oc_decode with OC_GATE_MASK); returns (1, d) in
    q's dtype."""
    kv = rows_layout(keys.unsqueeze(0), values.unsqueeze(0))
    p = N.OcDecodeParams()
    device = require_gpu(q, keys, values)
    qq = q.contiguous()
    out = torch.empty((1, kv.head_dim), dtype=q.dtype, device=device)
    p.kv = kv.struct()
    p.q, p.q_dtype, p.G, p.q_row_stride = qq.data_ptr(), dtype_code(qq.dtype, "q", allow_fp8=False), 1, qq.stride(0)
    p.gate, p.mode = N.OC_GATE_MASK, N.OC_MODE_CACHED
    p.tile_mask, p.tile_mask_row_stride = tile_mask.data_ptr(), tile_mask.stride(0)
    p.num_splits = auto_num_splits(kv.num_tiles, device)
    p.out_dtype = dtype_code(out.dtype, "out", allow_fp8=False)
    p.out, p.out_row_stride = out.data_ptr(), out.stride(0)
    stream = current_stream(device)
    lib = N.lib()
    need = lib.oc_decode_workspace_size(ctypes.byref(p))
    if need:
        ws = workspace(device, stream, need)
        p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    with torch.cuda.device(device):
        N.check("oc_decode", lib.oc_decode(ctypes.byref(p), ctypes.c_void_p(stream)))
    return out


def counts_metadata(keep: torch.Tensor, tiles_total: int) -> dict:
    retained = int(keep.sum().item())
    evicted = tiles_total - retained
    return {"tiles_retained": retained, "tiles_evicted": evicted,
            "eviction_rate": evicted / max(1, tiles_total)}


def kscale_mode(k_scale, num_rows: int, num_tiles: int, device) -> Tuple[int, float, Optional[torch.Tensor]]:
    """Scalar k_scale != 1 folds into q (reference semantics); a tensor of
    per-(row, tile) scales (extension) scales K elements."""
    if isinstance(k_scale, torch.Tensor):
        ks = k_scale.to(device=device, dtype=torch.float32).reshape(num_rows, -1)
        if ks.shape[1] < num_tiles:
            raise ValueError(f"k_scale has {ks.shape[1]} tiles per row, need {num_tiles}")
        return N.OC_KSCALE_TILE, 1.0, ks.contiguous()
    if k_scale != 1.0:
        return N.OC_KSCALE_Q_FOLD, float(k_scale), None
    return N.OC_KSCALE_NONE, 1.0, None


def vscale_mode(v_scale, num_rows: int, num_tiles: int, device) -> Tuple[int, Optional[torch.Tensor]]:
    if v_scale is None:
        return N.OC_VSCALE_NONE, None
    if not isinstance(v_scale, torch.Tensor):
        raise TypeError("v_scale must be a tensor of per-(row, tile) float32 scales")
    vs = v_scale.to(device=device, dtype=torch.float32).reshape(num_rows, -1)
    if vs.shape[1] < num_tiles:
        raise ValueError(f"v_scale has {vs.shape[1]} tiles per row, need {num_tiles}")
    return N.OC_VSCALE_TILE, vs.contiguous()


# ------------------------------------------------------------ model hook

def row_norms(x: torch.Tensor, low_band: int = 0) -> torch.Tensor:
    """oc_row_norms over the last dimension of a (n0, n1, n2, d) view (any
    strides, last dimension contiguous): float32 (n0, n1, n2); low_band > 0
    gives the Walsh-subspace high part."""
    device = require_gpu(x)
    if x.dim() != 4:
        raise ValueError(f"row_norms expects a 4-d view, got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    n0, n1, n2, d = x.shape
    out = torch.empty((n0, n1, n2), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        N.check("oc_row_norms", N.lib().oc_row_norms(
            x.data_ptr(), dtype_code(x.dtype, "x", allow_fp8=False), n0, n1, n2, x.stride(0), x.stride(1),
            x.stride(2), d, low_band, out.data_ptr(), ctypes.c_void_p(current_stream(device))))
    return out


def kth_smallest(x: torch.Tensor, k: int) -> torch.Tensor:
    """oc_kth_smallest: the k-th smallest (0-based) of each row of a float32
    (rows, n) tensor of non-negative values."""
    device = require_gpu(x)
    if x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1:
        x = x.to(torch.float32).contiguous().reshape(x.shape[0], -1)
    rows, n = x.shape
    out = torch.empty((rows,), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        N.check("oc_kth_smallest", N.lib().oc_kth_smallest(
            x.data_ptr(), rows, n, x.stride(0), k, out.data_ptr(), ctypes.c_void_p(current_stream(device))))
    return out


def group_gate(q_norms: torch.Tensor, k_norms: torch.Tensor, num_kv_heads: int, G: int, num_tiles: int,
               mask_cols: int, tau_norm: float, reduce: int, keep_polarity: bool = False, want_stats: bool = False):
    """oc_group_gate.  q_norms: float32 (batch, num_kv_heads * G); k_norms:
    float32 (batch or 1, num_kv_heads, >= num_tiles) (a batch of 1 is shared
    by every batch entry).  Returns (mask uint8 (batch, num_kv_heads,
    mask_cols), group norms float32 (batch, num_kv_heads)), plus with
    want_stats float32 (batch, num_kv_heads, 3): evicted complete tiles, the
    group norm and the largest K norm of the complete tiles (NaN if one is
    NaN, -inf if there are none)."""
    device = require_gpu(q_norms, k_norms)
    B = q_norms.shape[0]
    q_norms = q_norms.to(torch.float32).contiguous()
    if q_norms.numel() != B * num_kv_heads * G:
        raise ValueError(f"q_norms must hold {B} x {num_kv_heads * G} values")
    if (k_norms.dtype != torch.float32 or k_norms.dim() != 3 or k_norms.shape[1] != num_kv_heads
            or k_norms.shape[2] < num_tiles or k_norms.stride(2) != 1 or k_norms.shape[0] not in (1, B)):
        raise ValueError(f"k_norms must be a float32 (batch or 1, {num_kv_heads}, >= {num_tiles}) tensor")
    ksb = 0 if k_norms.shape[0] == 1 else k_norms.stride(0)
    mask = torch.empty((B, num_kv_heads, max(mask_cols, 1)), dtype=torch.uint8, device=device)
    gn = torch.empty((B, num_kv_heads), dtype=torch.float32, device=device)
    st = torch.empty((B, num_kv_heads, 3), dtype=torch.float32, device=device) if want_stats else None
    with torch.cuda.device(device):
        N.check("oc_group_gate", N.lib().oc_group_gate(
            q_norms.data_ptr(), B, num_kv_heads, G, reduce, k_norms.data_ptr(), ksb, k_norms.stride(1),
            num_tiles, mask_cols, float(tau_norm), 1 if keep_polarity else 0, mask.data_ptr(), mask.stride(0),
            mask.stride(1), gn.data_ptr(), _ptr(st), ctypes.c_void_p(current_stream(device))))
    return (mask, gn, st) if want_stats else (mask, gn)


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, tile_mask: Optional[torch.Tensor] = None,
                      scale: Optional[float] = None, want_entropy: bool = False, split: bool = True
                      ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """oc_prefill_attention: causal GQA attention of q (B, Hq, Sq, d) over k, v
    (B, Hkv, Skv, d) (last dimensions contiguous, other strides free),
    skipping the tiles whose tile_mask (B, Hkv, >= Skv // 64) byte is set.
    Returns (out (B, Hq, Sq, d) in q's dtype, entropy float32 (B, Hq, Sq) or
    None).  split: let the library run the longest causal windows as two
    workgroups each when the call fits the device in one round (it then uses
    the stream's workspace)."""
    device = require_gpu(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"q (B, Hq, Sq, d) and k, v (B, Hkv, Skv, d) expected, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, Hq, Sq, d = q.shape
    if k.shape[0] != B or k.shape[3] != d or Hq % k.shape[1]:
        raise ValueError(f"k {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k and v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    q, k, v = (_ready16(t) for t in (q, k, v))
    Hkv, Skv = k.shape[1], k.shape[2]
    out = torch.empty((B, Hq, Sq, d), dtype=q.dtype, device=device)
    ent = torch.empty((B, Hq, Sq), dtype=torch.float32, device=device) if want_entropy else None
    p = N.OcPrefillParams()
    p.q, (p.q_stride_b, p.q_stride_h, p.q_stride_s) = q.data_ptr(), q.stride()[:3]
    p.k, (p.k_stride_b, p.k_stride_h, p.k_stride_s) = k.data_ptr(), k.stride()[:3]
    p.v, (p.v_stride_b, p.v_stride_h, p.v_stride_s) = v.data_ptr(), v.stride()[:3]
    p.out, (p.out_stride_b, p.out_stride_h, p.out_stride_s) = out.data_ptr(), out.stride()[:3]
    p.dtype = dtype_code(q.dtype, "q", allow_fp8=False)
    p.batch, p.num_q_heads, p.num_kv_heads, p.q_len, p.kv_len, p.head_dim = B, Hq, Hkv, Sq, Skv, d
    if tile_mask is not None:
        if (tile_mask.dtype != torch.uint8 or tile_mask.dim() != 3 or tile_mask.shape[:2] != (B, Hkv)
                or tile_mask.stride(2) != 1 or tile_mask.device != device):
            raise ValueError(f"tile_mask must be a uint8 ({B}, {Hkv}, tiles) tensor on {device}")
        p.tile_mask, p.tile_mask_stride_b, p.tile_mask_stride_h = (tile_mask.data_ptr(), tile_mask.stride(0),
                                                                   tile_mask.stride(1))
        p.tile_mask_cols = tile_mask.shape[2]
    p.scale = float(scale) if scale is not None else 1.0 / (d ** 0.5)
    p.entropy = _ptr(ent)
    with torch.cuda.device(device):
        lib = N.lib()
        stream = current_stream(device)
        # a workspace lets the longest causal windows split over two workgroups
        nws = lib.oc_prefill_workspace_size(ctypes.byref(p)) if split else 0
        if nws:
            ws = workspace(device, stream, nws)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
        N.check("oc_prefill_attention", lib.oc_prefill_attention(ctypes.byref(p), ctypes.c_void_p(stream)))
    return out, ent


def _ready16(t: torch.Tensor) -> torch.Tensor:
    """t itself when its last dimension is contiguous and its base and every
    other stride are 16-byte aligned (the kernels' vector loads), else a
    contiguous copy."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


# ------------------------------------------------------------ 512-token spectra

SPECTRA_BLOCK = 512


def block_spectra(keys: torch.Tensor, q: Optional[torch.Tensor] = None, *, want_bounds: bool = False,
                  want_mean: bool = False, want_qnorm: bool = False) -> Dict[str, torch.Tensor]:
    """oc_block_spectra over the complete 512-token blocks of keys (S, H, d)
    (last dimension contiguous).  Returns float32 tensors e_low, e_mid,
    e_high, zeta, e_ac, energy (num_blocks, H); block_mean (num_blocks, H,
    d) with want_mean; with q (Sq, H, d): max_bound (num_blocks, H),
    with want_bounds bounds (Sq, num_blocks, H), with want_qnorm
    q_norm_max (H,) = max over queries of ||q_s||."""
    device = require_gpu(keys) if q is None else require_gpu(keys, q)
    if keys.dim() != 3:
        raise ValueError(f"keys must be (seq_len, num_heads, head_dim), got {tuple(keys.shape)}")
    keys = _ready16(keys)
    S, H, d = keys.shape
    nb = S // SPECTRA_BLOCK
    f32 = dict(dtype=torch.float32, device=device)
    out = {name: torch.empty((nb, H), **f32) for name in ("e_low", "e_mid", "e_high", "zeta", "e_ac", "energy")}
    p = N.OcSpectraParams()
    p.k, p.dtype = keys.data_ptr(), dtype_code(keys.dtype, "keys", allow_fp8=False)
    p.num_blocks, p.num_heads, p.head_dim, p.block_size = nb, H, d, SPECTRA_BLOCK
    p.k_token_stride, p.k_head_stride = keys.stride(0), keys.stride(1)
    for name, t in out.items():
        setattr(p, name, t.data_ptr())
    if want_mean:
        out["block_mean"] = torch.empty((nb, H, d), **f32)
        p.block_mean = out["block_mean"].data_ptr()
    if q is not None:
        if q.dim() != 3 or q.shape[1:] != (H, d):
            raise ValueError(f"q must be (seq_len_q, {H}, {d}), got {tuple(q.shape)}")
        if q.stride(-1) != 1:
            q = q.contiguous()
        p.q, p.q_dtype, p.q_len = q.data_ptr(), dtype_code(q.dtype, "q", allow_fp8=False), q.shape[0]
        p.q_token_stride, p.q_head_stride = q.stride(0), q.stride(1)
        out["max_bound"] = torch.empty((nb, H), **f32)
        p.max_bound = out["max_bound"].data_ptr()
        if want_bounds:
            out["bounds"] = torch.empty((q.shape[0], nb, H), **f32)
            p.bounds = out["bounds"].data_ptr()
        if want_qnorm:
            out["q_norm_max"] = torch.empty((H,), **f32)
            p.q_norm_max = out["q_norm_max"].data_ptr()
    with torch.cuda.device(device):
        N.check("oc_block_spectra", N.lib().oc_block_spectra(ctypes.byref(p),
                                                             ctypes.c_void_p(current_stream(device))))
    return out


def stream_compact(block_mask: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """oc_stream_compact: (indices int64 (n,), num_active int32 (1,)) on the device."""
    device = require_gpu(block_mask)
    m = block_mask.reshape(-1).to(torch.uint8).contiguous()
    n = m.numel()
    idx = torch.empty((n,), dtype=torch.int64, device=device)
    cnt = torch.zeros((1,), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        N.check("oc_stream_compact", N.lib().oc_stream_compact(
            m.data_ptr(), n, idx.data_ptr(), cnt.data_ptr(), ctypes.c_void_p(current_stream(device))))
    return idx, cnt


def compact_gate(spec: Dict[str, torch.Tensor], head_dim: int, tau: Optional[float], zeta_max: float,
                 underflow: float, tiles_per_block: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """oc_compact_gate on block_spectra(..., q, want_qnorm=True) outputs:
    (block mask uint8 (nb,), tile mask uint8 (nb * tiles_per_block,), stats
    float32 (9,): tau, zeta mean/std/min/max, retained, perfect,
    statistical, z_max)."""
    mb = spec["max_bound"]
    device = require_gpu(mb)
    nb, H = mb.shape
    bm = torch.empty((nb,), dtype=torch.uint8, device=device)
    tm = torch.empty((nb * tiles_per_block,), dtype=torch.uint8, device=device)
    st = torch.empty((9,), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        N.check("oc_compact_gate", N.lib().oc_compact_gate(
            mb.data_ptr(), spec["zeta"].data_ptr(), spec["energy"].data_ptr(), spec["q_norm_max"].data_ptr(),
            nb, H, head_dim, 0.0 if tau is None else float(tau), 1 if tau is None else 0, float(zeta_max),
            float(underflow), tiles_per_block, bm.data_ptr(), tm.data_ptr(), st.data_ptr(),
            ctypes.c_void_p(current_stream(device))))
    return bm, tm, st


def block_regimes(q: torch.Tensor, energy: torch.Tensor, head_dim: int, z_max, block_mask: torch.Tensor,
                  underflow: float, want_full: bool = False):
    """oc_block_regimes: per-block logit ceilings and eviction regimes.
    q (q_len, H, d) (its spatial row norms come from oc_row_norms), energy
    float32 (nb, H), z_max a number or a tensor (its largest element is
    used), block_mask bool/uint8 (nb,) or (nb, H).  Returns (regime int32
    (nb,), beta (nb,), gap (nb,), beta_full (nb, H) or None, counts int32 (3,)
    = perfect, statistical, retained)."""
    device = require_gpu(q, energy, block_mask)
    sq, H, d = q.shape
    qn = row_norms(q.reshape(1, 1, sq * H, d)).view(sq, H)
    energy = energy.to(torch.float32).contiguous()
    nb = energy.shape[0]
    if energy.dim() != 2 or energy.shape[1] != H:
        raise ValueError(f"block_energies must be (num_blocks, {H}), got {tuple(energy.shape)}")
    mask = block_mask.to(torch.uint8).contiguous()
    mask_heads = 1 if mask.dim() == 1 else mask.shape[-1]
    if mask.shape[0] != nb:
        raise ValueError(f"block_mask has {mask.shape[0]} blocks, block_energies {nb}")
    z_vec = None
    z_scalar = 0.0
    if isinstance(z_max, torch.Tensor) and z_max.dim() > 0:
        require_gpu(z_max)
        z_vec = z_max.to(torch.float32).contiguous().reshape(-1)
    else:
        z_scalar = float(z_max)
    regime = torch.empty((nb,), dtype=torch.int32, device=device)
    beta = torch.empty((nb,), dtype=torch.float32, device=device)
    gap = torch.empty((nb,), dtype=torch.float32, device=device)
    full = torch.empty((nb, H), dtype=torch.float32, device=device) if want_full else None
    counts = torch.empty((3,), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        N.check("oc_block_regimes", N.lib().oc_block_regimes(
            qn.data_ptr(), sq, H, energy.data_ptr(), nb, head_dim, z_scalar,
            None if z_vec is None else z_vec.data_ptr(), 0 if z_vec is None else z_vec.numel(),
            mask.data_ptr(), mask_heads, float(underflow), regime.data_ptr(), beta.data_ptr(), gap.data_ptr(),
            None if full is None else full.data_ptr(), counts.data_ptr(), ctypes.c_void_p(current_stream(device))))
    return regime, beta, gap, full, counts
