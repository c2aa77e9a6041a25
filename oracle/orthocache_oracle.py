"""CPU oracle for OrthoCache's spectral-gated decode attention.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP kernels
are compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``orthocache-gpu_amd/orthocache_gpu``) never does, and it never serves as a
fallback for the product path.

It restates, in numpy float32, the reference's CPU ("PyTorch fallback")
paths with the same per-head, per-tile loop structure:

* ``walsh_matrix``            <- fwht_fused_prototype.py:57-80
* ``fwht_scores``             <- fwht_fused_prototype.py:199-248
* ``fused_v1``                <- fused_eviction.py:460-549 (+ wrapper :698-755)
* ``fused_v2``                <- fused_eviction.py:380-457 (+ wrapper :573-628)
* ``gqa_v3``                  <- gqa_eviction.py:87-276    (+ wrapper :511-574)
* ``paged``                   <- paged_eviction.py:244-316 (+ wrapper :323-368)
* ``auto_num_splits``         <- fused_eviction.py:556-570
* ``dense_decode``            <- pipeline.py:558-568 (fp32 form)
* ``band_norm`` / ``band_norms`` <- SpectralNormCache.update_prefill /
                                 populate_from_keys (norm_cache.py:58-117)
* ``q_high_norm_exact``       <- compute_q_high_norm_exact (decode_gate.py:54-100)
* ``decode_gate``             <- decode_gate / _decode_gate_kernel
                                 (decode_gate.py:108-245); tight=True:
                                 _pytorch_decode_gate (decode_gate.py:248-295)
* ``apply_decode_mask``       <- apply_decode_mask(_vectorized) (decode_gate.py:302-374)
* ``block_sparse_attention``  <- _pytorch_block_sparse_attention (sparse_attention.py:144-203)
* ``indirect_attention``      <- _pytorch_indirect_attention (indirect_attention.py:136-197)
* ``hook_causal_attention``, ``hook_prefill``, ``hook_decode`` <- the
  model-side hook OrthoCache_GQA_Attention (eval/perplexity_eval.py:366-689
  of the reference tree: prefill branch :399-545, decode branch :575-673,
  dense fallback :675-689); ``torch_lower_median`` <- torch.median(dim)
  (:456); ``residual_tau`` / ``entropy_tau`` <- the governors (:236-318)
* ``fwht512``, ``block_spectra``, ``compact_forward`` <- the 512-token
  compact pipeline of orthocache_forward (fwht.py:6-45,
  spectral_energy.py:20-233, perfect_eviction.py:75-186,
  adaptive_attention.py:29-215, pipeline.py:458-583 of src/orthocache_gpu/)

(all paths relative to ``src/orthocache_gpu/triton_kernels/`` or
``src/orthocache_gpu/`` of the reference tree).

Extensions that the reference does not have (per-(row, tile) fp32 K/V
scales, per-sequence ``context_lens`` and GQA for the paged layout, the
cached-score gate and per-split partial states) are restated in the same
style and marked "extension" in their docstrings.

Pinning (how each function is checked, see tests/test_oracle.py):

* ``walsh_matrix``: closed form (-1)^popcount(i&j)/8, orthogonality,
  symmetry (the reference's own test_fused_kernel.py:45-92 properties).
* ``fwht_scores``: textbook radix-2 butterfly in float64, the closed forms
  E_high = 1/2 sum ||k_u - k_{u+32}||^2 and
  E_low = 1/8 sum_r ||S_r||^2 - 1/64 ||sum_t k_t||^2, integer-valued
  known-answer tiles (exact in any summation order), and golden vectors
  written by the reference's own CPU code (tests/golden/).
* ``fused_v1`` / ``fused_v2`` / ``gqa_v3`` / ``paged``: golden vectors
  from the reference, float64 brute-force softmax over the retained tokens,
  zero-eviction == dense, total eviction == 0.
* split partials: the LSE merge of the per-split partials equals the
  single-split result (float64), and the tile sets are {s + kP}.
* ``band_norm``: the closed forms of the [32,64) and [48,64) bands
  (1/2 sum ||k_u - k_{u+32}||^2 and 1/4 sum ||k_t - k_{t+16} - k_{t+32} +
  k_{t+48}||^2) in float64, integer tiles exact.
* ``q_high_norm_exact``: the residual of a least-squares projection onto
  block-constant vectors (float64), and its two special cases.
* ``decode_gate`` / ``apply_decode_mask``: explicit per-(head, tile) loops,
  special thresholds, and the max-over-G rule.
* ``block_sparse_attention`` / ``indirect_attention``: float64 softmax over
  the retained tokens, all blocks == dense, no block == zeros.
* hook functions: causal attention == per-query dense decode over the
  visible keys (float64), no eviction == causal softmax, entropy of uniform
  attention == ln n, the median rank rules on explicit lists, and the
  gate's decisions by an explicit per-(kv head, tile) loop
  (tests/test_oracle_hook.py).
* compact pipeline: fwht512 against the Sylvester matrix H512 / sqrt(512)
  and its involution, the band energies against closed forms (E_high =
  1/2 sum ||k_j - k_{j+256}||^2) and Parseval, constant blocks with zero AC
  energy, the bound >= every logit of the block (Cauchy-Schwarz), and
  stream compaction against torch.argsort (tests/test_oracle_compact.py).
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

TILE_SIZE = 64
BAND_LOW_64 = (1, 8)
BAND_HIGH_64 = (32, 64)

F32 = np.float32
_EPS_ZETA = F32(1e-6)          # `e_low + 1e-6` evaluated in float32
_M0 = F32(-1e9)                 # online-softmax initial max
_L_MIN = F32(1e-9)              # clamp(l, min=1e-9)
_CS_CLAMP = 1e-38               # subnormal clamp of the CS gate


# ---------------------------------------------------------------------------
# Walsh matrix and tile scores
# ---------------------------------------------------------------------------

def walsh_matrix(n: int = TILE_SIZE) -> np.ndarray:
    """Sylvester Hadamard matrix scaled by 1/sqrt(n), float32.

    Follows generate_walsh_matrix (fwht_fused_prototype.py:57-80):
    H_{2m} = [[H, H], [H, -H]], then H / n**0.5.
    """
    assert n > 0 and (n & (n - 1)) == 0, f"n must be a power of 2, got {n}"
    h = np.ones((1, 1), dtype=F32)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]]).astype(F32)
    return (h / F32(n ** 0.5)).astype(F32)


def _as_f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=F32))


def tile_energies(k_tile: np.ndarray, w: np.ndarray) -> Tuple[F32, F32]:
    """(E_low, E_high) of one 64xd fp32 tile: X = W @ K, row-energies summed
    over head_dim, bands [1,8) and [32,64) (fused_eviction.py:424-427)."""
    spec = w @ k_tile
    eps = np.sum(spec * spec, axis=1, dtype=F32)
    e_low = np.sum(eps[BAND_LOW_64[0]:BAND_LOW_64[1]], dtype=F32)
    e_high = np.sum(eps[BAND_HIGH_64[0]:BAND_HIGH_64[1]], dtype=F32)
    return F32(e_low), F32(e_high)


def zeta_of(e_low: F32, e_high: F32) -> F32:
    """zeta = e_high / (e_low + 1e-6) in float32 (fused_eviction.py:428)."""
    return F32(F32(e_high) / F32(F32(e_low) + _EPS_ZETA))


def fwht_scores(keys: np.ndarray, zeta_max: float, tile_size: int = TILE_SIZE):
    """Batched tile scores for a (num_tiles*64, d) key matrix.

    Follows _pytorch_fwht_eviction (fwht_fused_prototype.py:199-248):
    returns (keep mask [True = retain, zeta <= zeta_max], zeta, e_low, e_high).
    """
    keys = _as_f32(keys)
    n, d = keys.shape
    t = n // tile_size
    assert n == t * tile_size
    w = walsh_matrix(tile_size)
    tiles = keys.reshape(t, tile_size, d)
    spec = np.matmul(w[None], tiles)
    eps = np.sum(spec * spec, axis=2, dtype=F32)
    e_low = np.sum(eps[:, BAND_LOW_64[0]:BAND_LOW_64[1]], axis=1, dtype=F32)
    e_high = np.sum(eps[:, BAND_HIGH_64[0]:BAND_HIGH_64[1]], axis=1, dtype=F32)
    zeta = (e_high / (e_low + _EPS_ZETA)).astype(F32)
    keep = zeta.astype(np.float64) <= float(zeta_max)
    return keep, zeta, e_low, e_high


def cs_keep(e_high: F32, q_group: np.ndarray, tau: float) -> bool:
    """Cauchy-Schwarz gate of gqa_eviction.py:222-239.

    k_high_norm = ||X[32:64]||_F (0 if < 1e-38); q_norms = ||q_g||_2 (0 if
    < 1e-38); evicted iff max_g(q_norm_g * k_high_norm) <= tau.  The norm is
    taken as sqrt of the band energy (the Frobenius norm's definition).
    Returns True when the tile is retained.
    """
    kn = F32(np.sqrt(F32(e_high)))
    if float(kn) < _CS_CLAMP:
        kn = F32(0.0)
    qn = q_norms(q_group)
    cs = (qn * kn).astype(F32)
    mx = float(np.max(cs)) if cs.size else float("-inf")
    if math.isnan(mx):
        return True
    return not (mx <= float(tau))


def q_norms(q_group: np.ndarray) -> np.ndarray:
    """||q_g||_2 per row in float32 with the <1e-38 clamp (gqa_eviction.py:231-233)."""
    q = _as_f32(q_group)
    qn = np.sqrt(np.sum(q * q, axis=1, dtype=F32)).astype(F32)
    return np.where(qn < _CS_CLAMP, F32(0.0), qn).astype(F32)


# ---------------------------------------------------------------------------
# dtype helpers (the reference's q*k_scale is computed in q's dtype)
# ---------------------------------------------------------------------------

def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` ('f32', 'f16', 'bf16') with RNE and
    return them as float32."""
    x = _as_f32(x)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(F32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        nan = np.isnan(x)
        lsb = (u >> 16) & 1
        r = ((u + 0x7FFF + lsb) >> 16) << 16
        out = (r & 0xFFFFFFFF).astype(np.uint32).view(F32)
        return np.where(nan, x, out).astype(F32)
    raise ValueError(dtype)


def fp8_e4m3fn_table() -> np.ndarray:
    """float value of each of the 256 OCP e4m3fn codes (0x7f/0xff are NaN)."""
    out = np.zeros(256, dtype=F32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def fp8_encode(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest e4m3fn code (RNE, saturating at 448)."""
    table = fp8_e4m3fn_table()
    finite = np.where(np.isnan(table), np.inf, table)
    pos = np.argsort(finite[:128])
    vals = finite[:128][pos]
    x = _as_f32(x)
    ax = np.minimum(np.abs(x), F32(448.0))
    idx = np.searchsorted(vals, ax)
    idx = np.clip(idx, 1, len(vals) - 1)
    lo, hi = vals[idx - 1], vals[idx]
    code_lo, code_hi = pos[idx - 1], pos[idx]
    d_lo, d_hi = ax - lo, hi - ax
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (code_hi % 2 == 0))
    code = np.where(pick_hi, code_hi, code_lo).astype(np.uint8)
    code = np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)
    return code


# ---------------------------------------------------------------------------
# Online-softmax tile update (fused_eviction.py:434-445)
# ---------------------------------------------------------------------------

class _State:
    __slots__ = ("m", "l", "acc")

    def __init__(self, d: int):
        self.m = _M0
        self.l = F32(0.0)
        self.acc = np.zeros(d, dtype=F32)


def _update(st: _State, q_row: np.ndarray, k_tile: np.ndarray, v_tile: np.ndarray,
            scale: F32, valid: Optional[int] = None) -> None:
    logits = (k_tile @ q_row).astype(F32) * scale
    if valid is not None and valid < logits.shape[0]:
        logits = logits.copy()
        logits[valid:] = F32(-np.inf)
    local_max = F32(np.max(logits))
    new_max = F32(max(st.m, local_max)) if not np.isnan(local_max) else local_max
    p = np.exp((logits - new_max).astype(F32)).astype(F32)
    s = np.sum(p, dtype=F32)
    alpha = F32(np.exp(F32(st.m - new_max)))
    st.l = F32(st.l * alpha + s)
    st.acc = (st.acc * alpha + (p @ v_tile).astype(F32)).astype(F32)
    st.m = new_max


def _finish(st: _State) -> np.ndarray:
    return (st.acc / max(st.l, _L_MIN)).astype(F32)


def _scale_of(d: int) -> F32:
    return F32(1.0 / (d ** 0.5))


# ---------------------------------------------------------------------------
# Reference CPU paths
# ---------------------------------------------------------------------------

def fused_v1(q, keys, values, zeta_max: float, tile_size: int = TILE_SIZE,
             return_mask: bool = False, k_scale: float = 1.0, q_dtype: str = "f32"):
    """Single-head zeta-gated decode.

    Follows fused_orthocache_attention (fused_eviction.py:698-755) and its
    CPU body _pytorch_fused_orthocache_attention (:460-549).  `q` is the
    (1, d) query already decoded to float32; `q_dtype` names its storage
    dtype so that `q * k_scale` is rounded like the reference
    (fused_eviction.py:746-748).  Returns (out (1, d) float32, metadata).
    """
    q = _as_f32(q)
    if k_scale != 1.0:
        q = round_to(q * F32(k_scale), q_dtype)
    keys, values = _as_f32(keys), _as_f32(values)
    d = q.shape[-1]
    t_count = keys.shape[0] // tile_size
    w = walsh_matrix(tile_size)
    scale = _scale_of(d)
    st = _State(d)
    mask = np.zeros(t_count, dtype=bool)
    kept = ev = 0
    for t in range(t_count):
        kt = keys[t * tile_size:(t + 1) * tile_size]
        el, eh = tile_energies(kt, w)
        if float(zeta_of(el, eh)) > zeta_max:
            ev += 1
            continue
        mask[t] = True
        kept += 1
        _update(st, q[0], kt, values[t * tile_size:(t + 1) * tile_size], scale)
    meta = {"tiles_retained": kept, "tiles_evicted": ev,
            "eviction_rate": ev / max(1, t_count)}
    if return_mask:
        meta["eviction_mask"] = mask
    return _finish(st)[None, :], meta


def fused_v2(q, keys, values, zeta_max: float, tile_size: int = TILE_SIZE,
             k_scale: float = 1.0, q_dtype: str = "f32"):
    """Multi-head zeta-gated decode; q (H, d), keys/values (H, S, d).

    Follows fused_orthocache_attention_v2 (fused_eviction.py:573-628) and
    _pytorch_fused_orthocache_multihead (:380-457).  Returns (out (H, d)
    float32, metadata, keep mask (H, T))."""
    q = _as_f32(q)
    if k_scale != 1.0:
        q = round_to(q * F32(k_scale), q_dtype)
    keys, values = _as_f32(keys), _as_f32(values)
    h_count, s_len, d = keys.shape
    t_count = s_len // tile_size
    w = walsh_matrix(tile_size)
    scale = _scale_of(d)
    outs = []
    kept = ev = 0
    mask = np.zeros((h_count, t_count), dtype=bool)
    for h in range(h_count):
        st = _State(d)
        for t in range(t_count):
            kt = keys[h, t * tile_size:(t + 1) * tile_size]
            el, eh = tile_energies(kt, w)
            if float(zeta_of(el, eh)) > zeta_max:
                ev += 1
                continue
            kept += 1
            mask[h, t] = True
            _update(st, q[h], kt, values[h, t * tile_size:(t + 1) * tile_size], scale)
        outs.append(_finish(st))
    meta = {"tiles_retained": kept, "tiles_evicted": ev,
            "eviction_rate": ev / max(1, t_count * h_count)}
    return np.stack(outs), meta, mask


def gqa_v3(q, keys, values, tau: float, num_query_groups: int,
           tile_size: int = TILE_SIZE, k_scale: float = 1.0, q_dtype: str = "f32"):
    """GQA decode with the Cauchy-Schwarz gate; q (Hkv*G, d), K/V (Hkv, S, d).

    Follows fused_orthocache_attention_v3_gqa (gqa_eviction.py:511-574) and
    _pytorch_gqa_cauchy_schwarz_attention (:87-276): one gate decision per
    (kv head, tile) from max_g ||q_g|| * ||X[32:64]||_F <= tau, then a
    separate online softmax per query head g (:249-259).
    Returns (out (Hq, d) float32, metadata, keep mask (Hkv, T))."""
    q = _as_f32(q)
    if k_scale != 1.0:
        q = round_to(q * F32(k_scale), q_dtype)
    keys, values = _as_f32(keys), _as_f32(values)
    hkv, s_len, d = keys.shape
    g_count = num_query_groups
    assert q.shape[0] == hkv * g_count, (
        f"num_query_heads ({q.shape[0]}) != num_kv_heads ({hkv}) × G ({g_count})")
    t_count = s_len // tile_size
    w = walsh_matrix(tile_size)
    scale = _scale_of(d)
    outs = []
    kept = ev = 0
    mask = np.zeros((hkv, t_count), dtype=bool)
    for kv in range(hkv):
        qg = q[kv * g_count:(kv + 1) * g_count]
        sts = [_State(d) for _ in range(g_count)]
        for t in range(t_count):
            kt = keys[kv, t * tile_size:(t + 1) * tile_size]
            _, eh = tile_energies(kt, w)
            if not cs_keep(eh, qg, tau):
                ev += 1
                continue
            kept += 1
            mask[kv, t] = True
            vt = values[kv, t * tile_size:(t + 1) * tile_size]
            for g in range(g_count):
                _update(sts[g], qg[g], kt, vt, scale)
        outs.extend(_finish(s) for s in sts)
    meta = {"tiles_retained": kept, "tiles_evicted": ev,
            "eviction_rate": ev / max(1, t_count * hkv),
            "num_kv_heads": hkv, "num_query_groups": g_count,
            "gate_type": "cauchy_schwarz"}
    return np.stack(outs), meta, mask


def paged(q, k_cache, v_cache, block_tables, zeta_max: float,
          tile_size: int = TILE_SIZE, k_scale: float = 1.0, q_dtype: str = "f32",
          k_is_fp8: bool = False):
    """Paged zeta-gated decode; q (B, H, d), caches (NB, H, bs, d).

    Follows fused_orthocache_attention_paged (paged_eviction.py:323-368) and
    _pytorch_paged_orthocache_attention (:244-316): every sequence is read
    for max_blocks*bs tokens through its block-table row; an fp8 key cache
    is first converted to q's dtype and multiplied by k_scale in that dtype
    (:354-357).  `k_cache` holds the decoded float32 values of the stored
    elements.  Returns (out (B, H, d) float32, {}, keep mask (B, H, T))."""
    q = _as_f32(q)
    k_cache, v_cache = _as_f32(k_cache), _as_f32(v_cache)
    if k_is_fp8:
        k_cache = round_to(round_to(k_cache, q_dtype) * F32(k_scale), q_dtype)
        k_scale = 1.0
    if k_scale != 1.0:
        q = round_to(q * F32(k_scale), q_dtype)
    bt = np.asarray(block_tables, dtype=np.int64)
    b_count, h_count, d = q.shape
    bs = k_cache.shape[2]
    t_count = (bt.shape[1] * bs) // tile_size
    w = walsh_matrix(tile_size)
    scale = _scale_of(d)
    out = np.zeros((b_count, h_count, d), dtype=F32)
    mask = np.zeros((b_count, h_count, t_count), dtype=bool)
    for b in range(b_count):
        for h in range(h_count):
            kh = np.concatenate([k_cache[bt[b, j], h] for j in range(bt.shape[1])])
            vh = np.concatenate([v_cache[bt[b, j], h] for j in range(bt.shape[1])])
            st = _State(d)
            for t in range(t_count):
                kt = kh[t * tile_size:(t + 1) * tile_size]
                el, eh = tile_energies(kt, w)
                if float(zeta_of(el, eh)) > zeta_max:
                    continue
                mask[b, h, t] = True
                _update(st, q[b, h], kt, vh[t * tile_size:(t + 1) * tile_size], scale)
            out[b, h] = _finish(st)
    return out, {}, mask


def auto_num_splits(num_tiles: int, num_cus: Optional[int]) -> int:
    """P = min(#CU, max(1, T//4), T), and 1 off-device (fused_eviction.py:556-570)."""
    if num_cus is None:
        return 1
    return max(1, min(num_cus, max(1, num_tiles // 4), num_tiles))


# ---------------------------------------------------------------------------
# Generalised decode (extensions): GQA x {none, zeta, cs} gate x scales x
# context lengths x per-split partials.  With G=1 / gate='zeta' / no scales /
# full-length rows it reduces to fused_v2; with gate='cs' to gqa_v3.
# ---------------------------------------------------------------------------

def decode_rows(q, keys, values, *, gate: str, threshold: float, G: int,
                tile_size: int = TILE_SIZE, k_scales=None, v_scales=None,
                lengths: Optional[Sequence[int]] = None,
                num_splits: Optional[int] = None, want_partials: bool = False):
    """Extension: gated decode over `rows` independent (batch, kv-head) rows.

    q (rows*G, d) float32; keys/values (rows, S, d) float32 (decoded element
    values); k_scales/v_scales (rows, T) float32 or None: the tile's value is
    element * scale (one float32 multiply).  lengths[r] (tokens, <= S): only
    tiles fully inside the length are scored; a partial tail tile is always
    retained and its tokens past the length are masked out of the softmax.
    gate in {'none', 'zeta', 'cs'}.

    The tile loop follows the reference's per-tile order; when num_splits is
    given the tiles of split s are {s + kP} (fused_eviction.py:259) and the
    per-split partial states (m, l, acc) are returned as well.
    Returns dict(out (rows*G, d), keep (rows, T), e_low, e_high,
    retained, evicted, [M, L, ACC])."""
    q = _as_f32(q)
    keys, values = _as_f32(keys), _as_f32(values)
    rows, s_len, d = keys.shape
    t_count = s_len // tile_size
    w = walsh_matrix(tile_size)
    scale = _scale_of(d)
    p_count = 1 if num_splits is None else num_splits
    keep = np.zeros((rows, t_count), dtype=bool)
    e_low = np.zeros((rows, t_count), dtype=F32)
    e_high = np.zeros((rows, t_count), dtype=F32)
    m_out = np.full((rows * G, p_count), _M0, dtype=F32)
    l_out = np.zeros((rows * G, p_count), dtype=F32)
    acc_out = np.zeros((rows * G, p_count, d), dtype=F32)
    out = np.zeros((rows * G, d), dtype=F32)
    kept = ev = 0
    for r in range(rows):
        length = s_len if lengths is None else int(lengths[r])
        n_tiles = min(t_count, -(-length // tile_size))
        qg = q[r * G:(r + 1) * G]
        for s in range(p_count):
            sts = [_State(d) for _ in range(G)]
            for t in range(s, n_tiles, p_count):
                kt = keys[r, t * tile_size:(t + 1) * tile_size]
                vt = values[r, t * tile_size:(t + 1) * tile_size]
                if k_scales is not None:
                    kt = (kt * F32(k_scales[r, t])).astype(F32)
                if v_scales is not None:
                    vt = (vt * F32(v_scales[r, t])).astype(F32)
                valid = length - t * tile_size
                full = valid >= tile_size
                el, eh = tile_energies(kt, w) if full else (F32(0), F32(0))
                e_low[r, t], e_high[r, t] = el, eh
                if not full or gate == "none":
                    k_ok = True
                elif gate == "zeta":
                    k_ok = not (float(zeta_of(el, eh)) > threshold)
                elif gate == "cs":
                    k_ok = cs_keep(eh, qg, threshold)
                else:
                    raise ValueError(gate)
                keep[r, t] = k_ok
                if not k_ok:
                    ev += 1
                    continue
                kept += 1
                for g in range(G):
                    _update(sts[g], qg[g], kt, vt, scale,
                            valid=None if full else valid)
            for g in range(G):
                m_out[r * G + g, s] = sts[g].m
                l_out[r * G + g, s] = sts[g].l
                acc_out[r * G + g, s] = sts[g].acc
    for i in range(rows * G):
        out[i] = lse_merge(m_out[i], l_out[i], acc_out[i])
    res = {"out": out, "keep": keep, "e_low": e_low, "e_high": e_high,
           "retained": kept, "evicted": ev}
    if want_partials:
        res.update(M=m_out, L=l_out, ACC=acc_out)
    return res


def lse_merge(m: np.ndarray, l: np.ndarray, acc: np.ndarray) -> np.ndarray:
    """Sequential log-sum-exp merge of split partials (fused_eviction.py:316-373):
    m' = max, l = l*e^(m-m') + l_s*e^(m_s-m'), acc likewise; acc/max(l,1e-9)."""
    m_run, l_run, a_run = F32(m[0]), F32(l[0]), acc[0].astype(F32)
    for s in range(1, len(m)):
        nm = F32(max(m_run, F32(m[s])))
        a1 = F32(np.exp(F32(m_run - nm)))
        a2 = F32(np.exp(F32(F32(m[s]) - nm)))
        l_run = F32(l_run * a1 + F32(l[s]) * a2)
        a_run = (a_run * a1 + acc[s].astype(F32) * a2).astype(F32)
        m_run = nm
    return (a_run / max(l_run, _L_MIN)).astype(F32)


def dense_decode(q, keys, values) -> np.ndarray:
    """Dense softmax decode in float64 over every token (the comparator of
    pipeline.py:558-568 / profile_multihead.py:127-146); q (R, d), K/V (R, S, d)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    logits = np.einsum("rd,rsd->rs", q, k) / math.sqrt(q.shape[-1])
    logits -= logits.max(axis=1, keepdims=True)
    p = np.exp(logits)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("rs,rsd->rd", p, v)


def fwht64_butterfly(x: np.ndarray) -> np.ndarray:
    """Textbook radix-2 FWHT along axis 0 in float64, natural (Sylvester)
    order, scaled by 1/8: the six-stage butterfly of
    test_fused_kernel.py:103-139."""
    x = np.array(x, dtype=np.float64)
    n = x.shape[0]
    h = 1
    while h < n:
        y = x.reshape(n // (2 * h), 2, h, *x.shape[1:])
        a, b = y[:, 0].copy(), y[:, 1].copy()
        y[:, 0], y[:, 1] = a + b, a - b
        x = y.reshape(x.shape)
        h *= 2
    return x / math.sqrt(n)


# ---------------------------------------------------------------------------
# Score-cache maintenance and the O(1) decode gate
# ---------------------------------------------------------------------------

def band_norm(k_tile: np.ndarray, band_lo: int = 48, band_hi: int = 64) -> F32:
    """||(W @ k_tile)[band_lo:band_hi]||_F of one 64xd tile in float32, 0
    below 1e-38 (SpectralNormCache.update_prefill, norm_cache.py:78-86)."""
    x = (walsh_matrix() @ _as_f32(k_tile)).astype(F32)
    n = F32(np.sqrt(np.sum(x[band_lo:band_hi] * x[band_lo:band_hi], dtype=F32)))
    return F32(0.0) if float(n) < _CS_CLAMP else n


def band_norms(keys: np.ndarray, band_lo: int = 48, band_hi: int = 64) -> np.ndarray:
    """band_norm of every complete tile of (rows, S, d) keys, (rows, S // 64)
    (populate_from_keys, norm_cache.py:90-117)."""
    keys = _as_f32(keys)
    rows, s_len, _ = keys.shape
    t_count = s_len // TILE_SIZE
    out = np.zeros((rows, t_count), dtype=F32)
    for r in range(rows):
        for t in range(t_count):
            out[r, t] = band_norm(keys[r, t * TILE_SIZE:(t + 1) * TILE_SIZE], band_lo, band_hi)
    return out


def q_high_norm_exact(q: np.ndarray, low_band: int = 8) -> np.ndarray:
    """sqrt(max(||q||^2 - sum_i S_i^2 / bs, 0)) over the last axis, float32,
    S_i the sums of low_band blocks of bs = d / low_band elements
    (compute_q_high_norm_exact, decode_gate.py:86-100)."""
    q = _as_f32(q)
    d = q.shape[-1]
    bs = d // low_band
    assert d % low_band == 0
    sq = np.sum(q * q, axis=-1, dtype=F32)
    sums = np.sum(q.reshape(*q.shape[:-1], low_band, bs), axis=-1, dtype=F32)
    lo = (np.sum(sums * sums, axis=-1, dtype=F32) / F32(bs)).astype(F32)
    hi = (sq - lo).astype(F32)
    hi = np.where(hi < 0, F32(0.0), hi)
    return np.sqrt(hi).astype(F32)


def decode_gate(q: np.ndarray, norm_cache: np.ndarray, tau: float, num_tiles: int, G: int,
                tile_size: int = TILE_SIZE, tight: bool = False, low_band: int = 8):
    """(mask (Hkv, max_tiles) bool True = evict, q_norms (Hkv,)).

    tight=False follows the GPU path (_decode_gate_kernel,
    decode_gate.py:140-181): the largest ||q_g||^2 of the group, then its
    square root.  tight=True follows _pytorch_decode_gate (:248-295): the
    largest Walsh-subspace ||q_high||.  Evict tile t < num_tiles of kv head h
    iff qn[h] * norm_cache[h, t] <= tau * tile_size * head_dim (float32)."""
    q = _as_f32(q)
    hq, d = q.shape
    hkv = hq // G
    nc = _as_f32(norm_cache)
    max_tiles = nc.shape[1]
    tau_norm = F32(tau * float(tile_size * d))
    qn = np.zeros(hkv, dtype=F32)
    for h in range(hkv):
        group = q[h * G:(h + 1) * G]
        if tight:
            qn[h] = np.max(q_high_norm_exact(group, low_band))
        else:
            best = F32(0.0)
            for g in range(G):
                sq = np.sum(group[g] * group[g], dtype=F32)
                if sq > best:
                    best = sq
            qn[h] = np.sqrt(best)
    mask = np.zeros((hkv, max_tiles), dtype=bool)
    for h in range(hkv):
        for t in range(num_tiles):
            mask[h, t] = bool(F32(qn[h] * nc[h, t]) <= tau_norm)
    return mask, qn


def apply_decode_mask(logits: np.ndarray, mask: np.ndarray, G: int, tile_size: int = TILE_SIZE,
                      num_tiles: Optional[int] = None) -> np.ndarray:
    """logits (Hq, 1, S): -inf over every evicted tile (decode_gate.py:302-331),
    on a copy."""
    out = np.array(logits, copy=True)
    s_len = out.shape[2]
    if num_tiles is None:
        num_tiles = s_len // tile_size
    for kv_h in range(mask.shape[0]):
        for t in range(num_tiles):
            if mask[kv_h, t]:
                out[kv_h * G:(kv_h + 1) * G, :, t * tile_size:min((t + 1) * tile_size, s_len)] = -np.inf
    return out


# ---------------------------------------------------------------------------
# Mask-given single-query attention
# ---------------------------------------------------------------------------

def _block_online_softmax(q, keys, values, blocks, block_size):
    """The per-block online softmax of the reference's CPU paths, float32."""
    q = _as_f32(q).reshape(1, -1)
    keys, values = _as_f32(keys), _as_f32(values)
    d = q.shape[1]
    scale = F32(1.0 / (d ** 0.5))
    m = _M0
    l = F32(0.0)
    acc = np.zeros((1, d), dtype=F32)
    for b in blocks:
        k = keys[b * block_size:(b + 1) * block_size]
        v = values[b * block_size:(b + 1) * block_size]
        logits = ((q @ k.T) * scale).astype(F32)
        new_m = F32(max(m, logits.max()))
        p = np.exp(logits - new_m).astype(F32)
        a = F32(np.exp(F32(m - new_m)))
        l = F32(l * a + p.sum(dtype=F32))
        acc = (acc * a + p @ v).astype(F32)
        m = new_m
    return (acc / max(l, _L_MIN)).astype(F32)


def block_sparse_attention(q, keys, values, block_mask, block_size: int = 512) -> np.ndarray:
    """Blocks b with block_mask[b], in order (sparse_attention.py:144-203); (1, d)."""
    n_blocks = keys.shape[0] // block_size
    return _block_online_softmax(q, keys, values, [b for b in range(n_blocks) if block_mask[b]], block_size)


def indirect_attention(q, keys, values, active_indices, num_active: int, block_size: int = 512) -> np.ndarray:
    """Blocks active_indices[:num_active], in list order (indirect_attention.py:136-197); (1, d)."""
    if num_active == 0:
        return np.zeros((1, np.asarray(q).shape[-1]), dtype=F32)
    return _block_online_softmax(q, keys, values, [int(b) for b in active_indices[:num_active]], block_size)


# ---------------------------------------------------------------- model hook
# eval/perplexity_eval.py of the reference tree

HOOK_HIGH_BAND = (48, 64)  # (tile_size * 3) // 4 .. tile_size (perplexity_eval.py:441-442)
_P_CLAMP = 1e-10           # attn_weights.clamp(min=1e-10) before the log (:526)


def torch_lower_median(x: np.ndarray) -> np.ndarray:
    """torch.median(dim=-1): the lower of the two middle values, rank
    (n - 1) // 2 of the sorted order (perplexity_eval.py:456)."""
    n = x.shape[-1]
    return np.sort(x, axis=-1)[..., (n - 1) // 2]


def residual_tau(tau: float, alpha: float, rates) -> float:
    """ResidualGovernor.get_tau_effective after the layers' rates were
    reported (perplexity_eval.py:270-276)."""
    return tau * max(0.0, 1.0 - alpha * float(sum(rates)))


def entropy_tau(tau: float, alpha: float, rates, beta: float, h_median: float, entropy) -> float:
    """EntropyGovernor.get_tau_effective (perplexity_eval.py:304-318)."""
    t = residual_tau(tau, alpha, rates)
    if entropy is not None:
        t *= 2.0 * (1.0 / (1.0 + np.exp(-beta * (entropy - h_median))))
    return t


def hook_tile_norms(keys: np.ndarray) -> np.ndarray:
    """||(H64 K_t)[48:64]||_F of every complete tile of (B, Hkv, S, d) keys,
    float32 (B, Hkv, S // 64) (perplexity_eval.py:466-470).  The hook's
    Walsh matrix is its own, unnormalised Sylvester H64 with entries +-1
    (generate_walsh_matrix, perplexity_eval.py:54-64), 8 x W64, so these
    norms are 8x the SpectralNormCache band norms of the same tiles."""
    B, H, S, _ = keys.shape
    T = S // TILE_SIZE
    out = np.zeros((B, H, T), dtype=F32)
    w = walsh_matrix() * F32(8.0)  # exact: +-1/8 -> +-1
    for b in range(B):
        for h in range(H):
            for t in range(T):
                x = (w @ _as_f32(keys[b, h, t * TILE_SIZE:(t + 1) * TILE_SIZE])).astype(F32)
                hi = x[HOOK_HIGH_BAND[0]:HOOK_HIGH_BAND[1]]
                out[b, h, t] = np.sqrt(np.sum(hi * hi, dtype=F32))
    return out


def hook_causal_attention(q, k, v, G: int, evict: Optional[np.ndarray] = None):
    """Causal GQA softmax attention in float64 with evicted tiles masked for
    every query of the group (perplexity_eval.py:418-430, :483-500, :533):
    query s of q (B, Hq, Sq, d) sees keys j <= s + Skv - Sq of k, v
    (B, Hkv, Skv, d); evict (B, Hkv, >= Skv // 64) bool covers the complete
    tiles.  A query with no key left gets zeros (nan_to_num).  Returns
    (out float64 (B, Hq, Sq, d), entropy float64 (B, Hq, Sq) of the
    1e-10-clamped probabilities over all Skv keys)."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    B, Hq, Sq, d = q.shape
    Skv = k.shape[2]
    T = Skv // TILE_SIZE
    scale = 1.0 / np.sqrt(d)
    out = np.zeros((B, Hq, Sq, d))
    ent = np.zeros((B, Hq, Sq))
    j = np.arange(Skv)
    for b in range(B):
        for h in range(Hq):
            logits = (q[b, h] @ k[b, h // G].T) * scale
            allowed = j[None, :] <= (np.arange(Sq)[:, None] + Skv - Sq)
            if evict is not None:
                tile_ok = np.ones(Skv, dtype=bool)
                for t in range(T):
                    if evict[b, h // G, t]:
                        tile_ok[t * TILE_SIZE:(t + 1) * TILE_SIZE] = False
                allowed = allowed & tile_ok[None, :]
            lg = np.where(allowed, logits, -np.inf)
            m = lg.max(axis=1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.where(allowed, np.exp(lg - m), 0.0)
            z = p.sum(axis=1, keepdims=True)
            p = np.where(z > 0, p / np.where(z > 0, z, 1.0), 0.0)
            out[b, h] = p @ v[b, h // G]
            pc = np.maximum(p, _P_CLAMP)
            ent[b, h] = -(pc * np.log(pc)).sum(axis=1)
    return out, ent


def hook_prefill(q, k, v, G: int, tau: float):
    """The prefill branch of OrthoCache_GQA_Attention.orthocache_attention
    for one call (perplexity_eval.py:399-545): per batch element and kv
    head, qn = max over the group of the lower median over positions of
    ||q||_2 (float32), k_norm = hook_tile_norms, and a complete tile is
    evicted when qn * k_norm / (64 d) <= tau (float64 compare).  Returns a
    dict: out (float64), evict (B, Hkv, T) bool, k_norms, qn (B, Hkv),
    per batch element `evicted`, `max_q`, `max_k`, `h_score`, `entropy`
    (the mean over heads and positions)."""
    q32 = _as_f32(q)
    B, Hq, Sq, d = q32.shape
    Hkv = k.shape[1]
    kn = hook_tile_norms(k)
    T = kn.shape[2]
    qnorm = np.sqrt(np.sum(q32.astype(np.float64) ** 2, axis=-1)).astype(F32)  # (B, Hq, Sq)
    med = torch_lower_median(qnorm)                                          # (B, Hq)
    qn = med.reshape(B, Hkv, G).max(axis=2)
    nf = float(TILE_SIZE * d)
    evict = np.zeros((B, Hkv, T), dtype=bool)
    for b in range(B):
        for h in range(Hkv):
            for t in range(T):
                evict[b, h, t] = (float(qn[b, h]) * float(kn[b, h, t])) / nf <= tau
    out, ent = hook_causal_attention(q, k, v, G, evict)
    max_q = np.maximum(qn.max(axis=1).astype(np.float64), 0.0)
    max_k = np.maximum(kn.reshape(B, -1).max(axis=1).astype(np.float64), 0.0) if T else np.zeros(B)
    return {"out": out, "evict": evict, "k_norms": kn, "qn": qn, "evicted": evict.reshape(B, -1).sum(axis=1),
            "max_q": max_q, "max_k": max_k, "h_score": max_q / (max_k + 1e-10),
            "entropy": ent.reshape(B, -1).mean(axis=1)}


def hook_decode(q, k, v, norm_cache: np.ndarray, G: int, tau: float, low_band: int = 8):
    """The decode branch (perplexity_eval.py:575-673): q (B, Hq, 1, d); per
    batch element and kv head, qn = element G // 2 of the sorted
    Walsh-subspace norms of the group's queries, and complete tile t is
    evicted when qn * norm_cache[kv, t] / (64 d) <= tau; the partial last
    tile is always attended.  Returns a dict: out (float64), evict,
    qn, skipped, max_q, max_k, h_score."""
    B, Hq, _, d = np.asarray(q).shape
    Hkv, Skv = k.shape[1], k.shape[2]
    T = Skv // TILE_SIZE
    qh = q_high_norm_exact(_as_f32(q)[:, :, 0], low_band)  # (B, Hq)
    qn = np.sort(qh.reshape(B, Hkv, G), axis=2)[:, :, G // 2]
    nf = float(TILE_SIZE * d)
    nc = _as_f32(norm_cache)
    evict = np.zeros((B, Hkv, T), dtype=bool)
    for b in range(B):
        for h in range(Hkv):
            for t in range(T):
                evict[b, h, t] = (float(qn[b, h]) * float(nc[h, t])) / nf <= tau
    out, _ = hook_causal_attention(q, k, v, G, evict)
    max_q = np.maximum(qn.max(axis=1).astype(np.float64), 0.0)
    max_k = np.full(B, max(0.0, float(nc[:Hkv, :T].max())) if T else 0.0)
    return {"out": out, "evict": evict, "qn": qn, "skipped": evict.reshape(B, -1).sum(axis=1),
            "max_q": max_q, "max_k": max_k, "h_score": max_q / (max_k + 1e-10)}


# ---------------------------------------------------------------- compact pipeline
# src/orthocache_gpu/ of the reference tree

COMPACT_BLOCK = 512
F32_UNDERFLOW = 88.72  # perfect_eviction.py:47


def fwht512(x: np.ndarray) -> np.ndarray:
    """Normalised natural-order 512-point Walsh-Hadamard transform along axis
    0 (fwht.py:6-45: nine radix-2 stages, each pairing the elements whose
    index differs in one bit, then / sqrt(512)), float64."""
    y = np.array(x, dtype=np.float64).copy()
    n = y.shape[0]
    assert n == COMPACT_BLOCK
    h = 1
    while h < n:
        y = y.reshape(n // (2 * h), 2, h, *y.shape[1:])
        a, b = y[:, 0].copy(), y[:, 1].copy()
        y[:, 0], y[:, 1] = a + b, a - b
        y = y.reshape(n, *y.shape[3:])
        h *= 2
    return y / math.sqrt(n)


def block_spectra(keys: np.ndarray, q: Optional[np.ndarray] = None):
    """Per 512-token block b and head h of keys (S, H, d): the band energies
    of fwht512 (spectral_energy.py:68-105; [1,64), [64,256), [256,512)),
    zeta = high / (low + 1e-6) (:108-137), AC energy (rows 1..511), spatial
    energy (:20-34), block mean = X[0] / sqrt(512), and with q (Sq, H, d)
    the query-aware bounds (:140-176) (Sq, nb, H) -- all float64."""
    k = np.asarray(keys, dtype=np.float64)
    S, H, d = k.shape
    nb = S // COMPACT_BLOCK
    out = {n: np.zeros((nb, H)) for n in ("e_low", "e_mid", "e_high", "zeta", "e_ac", "energy")}
    out["block_mean"] = np.zeros((nb, H, d))
    for b in range(nb):
        for h in range(H):
            blk = k[b * COMPACT_BLOCK:(b + 1) * COMPACT_BLOCK, h]
            X = fwht512(blk)
            e = np.sum(X * X, axis=1)
            out["e_low"][b, h] = e[1:64].sum()
            out["e_mid"][b, h] = e[64:256].sum()
            out["e_high"][b, h] = e[256:].sum()
            out["zeta"][b, h] = out["e_high"][b, h] / (out["e_low"][b, h] + 1e-6)
            out["e_ac"][b, h] = e[1:].sum()
            out["energy"][b, h] = np.sum(blk * blk)
            out["block_mean"][b, h] = X[0] / math.sqrt(COMPACT_BLOCK)
    if q is not None:
        qq = np.asarray(q, dtype=np.float64)
        align = np.einsum("qhd,bhd->qbh", qq, out["block_mean"]) / math.sqrt(d)
        resid = np.linalg.norm(qq, axis=-1)[:, None, :] * np.sqrt(out["e_ac"])[None] / math.sqrt(d)
        out["bounds"] = align + resid
        out["max_bound"] = out["bounds"].max(axis=0)
    return out


def compact_forward(q, keys, values, zeta_max: float = 5.0, tau: Optional[float] = None):
    """orthocache_forward(mode='compact') past the crossover bypass
    (pipeline.py:458-555): tau = mean - std (unbiased) of the max bounds
    when not given (:571-583); (block, head) retained iff max bound >= tau
    and zeta <= zeta_max (spectral_energy.py:198-233); a block is attended
    when any head retains it; every query attends every key of the attended
    blocks (adaptive_attention.py:46-91, online softmax from -1e30).
    Returns (out float64 (Sq, H, d), info dict: tau, block_mask, unified,
    retained, zeta stats, perfect / statistical counts)."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(keys, dtype=np.float64)
    v64 = np.asarray(values, dtype=np.float64)
    Sq, H, d = q64.shape
    spec = block_spectra(k64, q64)
    g = compact_gate(spec["max_bound"], spec["zeta"], spec["energy"], np.linalg.norm(q64, axis=-1).max(axis=0), d,
                     zeta_max, tau)
    tau, unified, retained = g["tau"], g["unified"], g["retained"]
    nb = unified.shape[0]
    out = np.zeros((Sq, H, d))
    if retained:
        keep = np.repeat(unified, COMPACT_BLOCK)
        for h in range(H):
            kk = k64[:nb * COMPACT_BLOCK, h][keep]
            vv = v64[:nb * COMPACT_BLOCK, h][keep]
            lg = q64[:, h] @ kk.T / math.sqrt(d)
            p = np.exp(lg - lg.max(axis=1, keepdims=True))
            out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vv
    return out, dict(g, spectra=spec)


def compact_gate(max_bound, zeta, energy, qmax, d: int, zeta_max: float, tau: Optional[float] = None):
    """The compact forward's gates and statistics from the (block, head)
    tables (pipeline.py:463-527): tau = mean - unbiased std of the max
    bounds when not given (:571-583); (block, head) kept iff max bound >= tau
    and zeta <= zeta_max (spectral_energy.py:198-233); a block is attended
    when any head keeps it; zeta statistics over the per-block head means
    (pipeline.py:482-487); z_max = the largest retained max bound, beta =
    max_h qmax_h sqrt(E) / sqrt(d), and an evicted block is perfect iff
    z_max - beta >= the float32 underflow margin (perfect_eviction.py:75-186).
    qmax (H,) is the largest query norm per head."""
    mb = np.asarray(max_bound, dtype=np.float64)
    zeta = np.asarray(zeta, dtype=np.float64)
    energy = np.asarray(energy, dtype=np.float64)
    qmax = np.asarray(qmax, dtype=np.float64)
    nb = mb.shape[0]
    if tau is None:
        tau = float(mb.mean() - mb.std(ddof=1))
    block_mask = (mb >= tau) & (zeta <= zeta_max)
    unified = block_mask.any(axis=1)
    retained = int(unified.sum())
    zah = zeta.mean(axis=1)
    z_max = float(mb[unified].max()) if retained else 0.0
    beta = (qmax[None, :] * np.sqrt(np.maximum(energy, 0.0)) / math.sqrt(d)).max(axis=1)
    gap = z_max - beta
    perfect = int(((~unified) & (gap >= F32_UNDERFLOW)).sum())
    statistical = int(((~unified) & (gap < F32_UNDERFLOW)).sum())
    return {"tau": tau, "block_mask": block_mask, "unified": unified, "retained": retained,
            "zeta_mean": float(zah.mean()), "zeta_std": float(zah.std(ddof=1)) if nb > 1 else float("nan"),
            "zeta_min": float(zah.min()), "zeta_max_observed": float(zah.max()), "z_max": z_max,
            "perfect": perfect, "statistical": statistical}


def block_regimes(q, energy, head_dim: int, z_max, block_mask, underflow: float = F32_UNDERFLOW):
    """Per-block ceiling, gap and regime in the reference's float32 arithmetic
    (perfect_eviction.py:75-186): qn_h = max over queries of ||q_s,h||;
    beta[b, h] = qn_h * sqrt(clamp(E, 0)) / float32(sqrt(d)); beta_b = max over
    h; gap = float32(z) - beta_b; regime 0 when any mask entry of the block is
    set, 1 when gap >= underflow, 2 when gap < underflow (NaN: 0, counted in
    neither).  z_max may be an array (its largest element).  Returns
    (regime int32, beta float32 (nb,), gap float32, beta_full float32 (nb, H),
    counts (perfect, statistical, retained))."""
    f32 = np.float32
    q = np.asarray(q, dtype=np.float32)
    qn = np.sqrt(np.sum(q.astype(np.float64) ** 2, axis=-1)).astype(f32).max(axis=0)
    e = np.asarray(energy, dtype=f32)
    full = (qn[None, :] * np.sqrt(np.maximum(e, f32(0)))) / f32(math.sqrt(head_dim))
    beta = full.max(axis=1) if full.shape[1] else np.zeros(full.shape[0], f32)
    z = f32(np.max(np.asarray(z_max, dtype=f32))) if np.ndim(z_max) else f32(z_max)
    gap = (z - beta).astype(f32)
    m = np.asarray(block_mask, dtype=bool)
    unified = m.any(axis=1) if m.ndim > 1 else m
    thr = f32(underflow)
    perfect = ~unified & (gap >= thr)
    statistical = ~unified & (gap < thr)
    regime = np.where(perfect, 1, np.where(statistical, 2, 0)).astype(np.int32)
    return regime, beta.astype(f32), gap, full.astype(f32), (int(perfect.sum()), int(statistical.sum()),
                                                              int(unified.sum()))


def stream_compact(mask: np.ndarray):
    """(active-first stable order, count) (adaptive_attention.py:29-43)."""
    mask = np.asarray(mask, dtype=bool)
    idx = [i for i in range(mask.size) if mask[i]] + [i for i in range(mask.size) if not mask[i]]
    return np.array(idx, dtype=np.int64), int(mask.sum())
