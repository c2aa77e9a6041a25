"""Model-side attention hook: drop-in equivalents of the reference's
OrthoCache_GQA_Attention, ResidualGovernor, EntropyGovernor and
patch_model_attention (eval/perplexity_eval.py:236-318, :320-741).

The hook sits where a decoder layer calls scaled-dot-product attention,
after the Q/K/V projections and RoPE, with q (batch, num_q_heads, q_len,
head_dim) and k, v (batch, num_kv_heads, kv_len, head_dim):

* kv_len < 64: causal attention, nothing gated (perplexity_eval.py:388-395).
* q_len == 1 with a populated SpectralNormCache: the decode branch
  (perplexity_eval.py:575-673).  Per (batch, kv head): the median of the
  group's Walsh-subspace q norms (rank G // 2 of their sorted order) times
  the cached ||K_high||_F of each complete tile, over 64 * head_dim, at or
  below tau evicts the tile; the surviving tiles (and the partial last
  tile) are attended by the split-K decode kernel (oc_decode with a tile
  mask), which never reads an evicted tile's K or V.
* otherwise the prefill branch (perplexity_eval.py:399-545): per q head the
  lower median over positions of ||q||_2, the max over the group, times the
  tile's ||(H64 K_t)[48:64]||_F (the unnormalised Walsh matrix of the
  reference's evaluation code) over 64 * head_dim, at or below tau evicts
  the tile for every query of the group; causal attention over the rest
  (oc_prefill_attention), the attention entropy when the governor reads
  it, and the band norms go to the norm cache.

Statistics, governor updates and norm-cache contents follow the reference
call for call (one entry per batch element per layer call).  The per-call
values are reduced on the GPU and reach the host when `stats` is read (one
transfer for all calls since the last read), or at once when a governor
needs them for the next layer's tau.  Differences, all keyword-only or
invisible at the reference's inputs:

* ``score_new_tiles=True`` scores the tiles that complete during decode
  into the norm cache, from each call's own K, before the gate reads them
  (the reference leaves them at 0, so its decode gate evicts them);
  default False, the reference behaviour.
* a key/value already expanded to num_q_heads heads (transformers' SDPA
  path when a mask is passed) is reduced to its distinct kv heads.
* the band norms come from the SpectralNormCache kernel, which clamps
  norms below 1e-38 to 0 where the reference's prefill does not; a float32
  norm is either 0 or above 3e-23, so the stored values are the same.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import _launch as X
from . import _native as N

TILE = 64
_HIGH_BAND = (48, 64)  # (tile_size * 3) // 4 .. tile_size (perplexity_eval.py:441-442)
_LOW_BAND = 8          # _compute_q_high_norm's default (perplexity_eval.py:547)
# The hook transforms with its own unnormalised Sylvester H64, entries +-1
# (perplexity_eval.py:54-64), which is 8 x the W64 = H64 / 8 of the band-norm
# kernel: every ||K_high||_F the hook forms (its gate, statistics and norm
# cache) is 8x the kernel's.  A power-of-two scale, so exact.
_HOOK_NORM_SCALE = 8.0


class ResidualGovernor:
    """tau_effective = tau_base * max(0, 1 - alpha * sum of the earlier layers'
    eviction rates) (perplexity_eval.py:236-276)."""

    def __init__(self, alpha: float = 0.5):
        self.alpha = alpha
        self.eps_accum = 0.0
        self.layer_history = []

    def reset(self):
        self.eps_accum = 0.0
        self.layer_history = []

    def get_tau_effective(self, tau_base: float) -> float:
        return tau_base * max(0.0, 1.0 - self.alpha * self.eps_accum)

    def report_layer(self, eviction_rate: float):
        self.layer_history.append(eviction_rate)
        self.eps_accum += eviction_rate


class EntropyGovernor(ResidualGovernor):
    """The residual governor's tau times 2 * sigmoid(beta * (H - h_median)),
    H the attention entropy of the current layer (perplexity_eval.py:279-318)."""

    def __init__(self, alpha: float = 0.5, beta: float = 1.0, h_median: float = 1.56):
        super().__init__(alpha=alpha)
        self.beta = beta
        self.h_median = h_median
        self.current_entropy = None

    def set_entropy(self, entropy: float):
        self.current_entropy = entropy

    def get_tau_effective(self, tau_base: float) -> float:
        tau = super().get_tau_effective(tau_base)
        if self.current_entropy is not None:
            tau *= 2.0 / (1.0 + math.exp(-self.beta * (self.current_entropy - self.h_median)))
        return tau


class _Stats(dict):
    """The hook's statistics (the reference's `stats` dict).  Each call's
    values are reduced on the GPU and wait here as device tensors with the
    function that folds them in; the first read of the dict moves all waiting
    values to the host in one transfer and folds them in call order, so a
    patched model's forward does not stop for them.  A governor needs each
    layer's eviction rate before the next layer's tau, so with a governor
    every call folds at once."""

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        self._pending = []
        self._folding = False
        self._rings = {}  # (device, shape): views of a (_MAX_PENDING,) + shape float32 device ring
        self._ring_next = 0

    def ring_rows(self, device: torch.device, shape: tuple) -> torch.Tensor:
        """float32 device values of one call, of the given shape, to be
        deferred: a slot of a ring that is free again once the pending calls
        are folded (at most _MAX_PENDING of them), so that a call allocates
        nothing.  The slots' views are made once."""
        if self._ring_next >= self._MAX_PENDING:
            # (only after calls that failed before deferring) no pending call
            # holds a row once the pending calls are folded
            self.fold()
            self._ring_next = 0
        key = (device, shape)
        views = self._rings.get(key)
        if views is None:
            ring = torch.empty((self._MAX_PENDING,) + tuple(shape), dtype=torch.float32, device=device)
            views = self._rings[key] = list(ring.unbind(0))
        slot = self._ring_next
        self._ring_next += 1
        return views[slot]

    _MAX_PENDING = 256  # calls held before a fold (bounds the device tensors kept alive)

    def defer(self, fold, dev: torch.Tensor, run=None) -> None:
        """fold(host) folds one call's values (dev as a float64 array of its
        shape).  run = (key, fold_many): consecutive calls with equal keys
        fold together, fold_many(host of shape (n,) + dev.shape) standing for
        their n folds in call order."""
        self._pending.append((fold, dev, run))
        if len(self._pending) >= self._MAX_PENDING:
            self.fold()

    def fold(self) -> None:
        if not self._pending or self._folding:
            return
        pending, self._pending = self._pending, []
        self._ring_next = 0  # the transfer below completes every pending call's writes
        # one device concatenation (the values are float32), one transfer,
        # then float64 numpy on the host: the folds index it per call, where
        # numpy's scalar ops cost a fraction of torch's
        host = torch.cat([d.reshape(-1) for _, d, _ in pending]).cpu().numpy().astype(np.float64)
        self._folding = True
        try:
            i = j = 0
            while j < len(pending):
                fn, d, run = pending[j]
                k = j + 1
                if run is not None:
                    while k < len(pending) and pending[k][2] is not None and pending[k][2][0] == run[0]:
                        k += 1
                n, size = k - j, d.numel()
                if n > 1:
                    run[1](host[i:i + n * size].reshape((n,) + tuple(d.shape)))
                else:
                    fn(host[i:i + size].reshape(tuple(d.shape)))
                i += n * size
                j = k
        finally:
            self._folding = False


def _folding(name):
    base = getattr(dict, name)

    def method(self, *args, **kw):
        self.fold()
        return base(self, *args, **kw)
    method.__name__ = name
    return method


for _name in ('__getitem__', '__setitem__', '__delitem__', '__contains__', '__iter__', '__len__', '__repr__',
              '__eq__', 'get', 'keys', 'values', 'items', 'copy', 'pop', 'popitem', 'setdefault', 'update'):
    setattr(_Stats, _name, _folding(_name))


def _empty_stats() -> dict:
    return _Stats({
        'total_tiles': 0, 'evicted_tiles': 0, 'layers_processed': 0, 'cs_bounds': [],
        'hallucination_scores': [], 'q_search_intensity': [], 'k_info_density': [],
        'decode_steps': 0, 'decode_tiles_skipped': 0, 'decode_tiles_total': 0,
    })


class OrthoCache_GQA_Attention:
    """Cauchy-Schwarz spectral gate + attention in place of a decoder layer's
    SDPA call (perplexity_eval.py:320-689).  All device work runs in
    liborthocache_hip; the class keeps the reference's attributes
    (tau, verbose, governor, norm_cache, stats) and methods."""

    def __init__(self, tau: float = 1.0, verbose: bool = False,
                 governor: Optional[ResidualGovernor] = None, *, score_new_tiles: bool = False):
        self.tau = tau
        self.verbose = verbose
        self.governor = governor
        self.norm_cache = None
        self.score_new_tiles = score_new_tiles
        self._prefill_tiles = 0  # complete tiles of the last prefill
        self.stats = _empty_stats()

    def reset_stats(self):
        self.stats = _empty_stats()

    @property
    def eviction_rate(self) -> float:
        if self.stats['total_tiles'] == 0:
            return 0.0
        return self.stats['evicted_tiles'] / self.stats['total_tiles']

    # ------------------------------------------------------------ dispatch

    def orthocache_attention(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                             num_query_groups: int) -> torch.Tensor:
        """(batch, num_q_heads, q_len, head_dim) attention output in query's
        dtype (perplexity_eval.py:366-545)."""
        key, value = _distinct_kv(query, key, value, num_query_groups)
        q_len, kv_len = query.shape[2], key.shape[2]
        if kv_len < TILE:
            return self._dense_attention(query, key, value, num_query_groups)
        if q_len == 1 and self.norm_cache is not None and self.norm_cache.is_populated:
            return self._decode_attention(query, key, value, num_query_groups)
        return self._prefill_attention(query, key, value, num_query_groups)

    def _tau(self) -> float:
        return self.governor.get_tau_effective(self.tau) if self.governor is not None else self.tau

    # ------------------------------------------------------------ prefill

    def _prefill_attention(self, query, key, value, G):
        B, Hq, Sq, d = query.shape
        Hkv, Skv = key.shape[1], key.shape[2]
        T = Skv // TILE
        tau = self._tau()
        # ||(H64 K_t)[48:64]||_F of every complete tile, (B, Hkv, T)
        kn = torch.empty((B * Hkv, T), dtype=torch.float32, device=key.device)
        X.band_norms(X.rows_layout(key.reshape(B * Hkv, Skv, d), None), 0, T, _HIGH_BAND, kn)
        kn = kn.view(B, Hkv, T).mul_(_HOOK_NORM_SCALE)
        # per q head: lower median over positions of ||q||_2; the group's max
        med = X.kth_smallest(X.row_norms(query).view(B * Hq, Sq), (Sq - 1) // 2).view(B, Hq)
        evict, qn = X.group_gate(med, kn, Hkv, G, T, T, tau * TILE * d, N.OC_GROUP_MAX)
        want_entropy = self.governor is not None and hasattr(self.governor, 'set_entropy')
        out, ent = X.prefill_attention(query, key, value, tile_mask=evict, want_entropy=want_entropy)
        if self.norm_cache is not None:
            self._store_norms(kn[B - 1], Hkv, T)
        self._prefill_tiles = T
        # per batch element [evicted, max q norm, max k norm, mean entropy], reduced on the GPU
        zeros = torch.zeros((B,), dtype=torch.float32, device=query.device)
        dev = torch.stack([
            evict.view(B, -1).sum(1, dtype=torch.int64).to(torch.float32),
            qn.amax(1).clamp(min=0.0),
            kn.reshape(B, -1).amax(1).clamp(min=0.0),
            ent.view(B, -1).mean(1) if ent is not None else zeros,
        ])
        stats, gov = self.stats, self.governor

        def fold(host):
            for b in range(B):
                evicted = int(host[0, b])
                _add(stats, 'total_tiles', Hkv * T)
                _add(stats, 'evicted_tiles', evicted)
                _exhaust(stats, float(host[1, b]), float(host[2, b]))
                if gov is not None and Hkv * T > 0:
                    gov.report_layer(evicted / (Hkv * T))
                if want_entropy:
                    gov.set_entropy(float(host[3, b]))
                    _dset(stats, 'entropy', float(host[3, b]))
            _add(stats, 'layers_processed', 1)
        stats.defer(fold, dev)
        if gov is not None:
            stats.fold()
        return out

    def _store_norms(self, kn_last: torch.Tensor, Hkv: int, T: int) -> None:
        """The reference's per-batch loop writes cache[kv_h, t] for every batch
        element in turn, so the last one's norms remain (perplexity_eval.py:472-477)."""
        nc = self.norm_cache
        if Hkv > nc.num_kv_heads or T > nc.max_tiles:
            raise IndexError(f"norm cache ({nc.num_kv_heads} heads x {nc.max_tiles} tiles) is smaller than the "
                             f"prefill ({Hkv} heads x {T} tiles)")
        nc.cache[:Hkv, :T].copy_(kn_last)
        nc.valid_tiles[:Hkv].clamp_(min=T)
        nc._populated = True


    # ------------------------------------------------------------ decode

    def _compute_q_high_norm(self, q_vec: torch.Tensor, low_band: int = _LOW_BAND) -> float:
        """||q_high||_2 of one head_dim vector (perplexity_eval.py:547-573)."""
        return float(X.row_norms(q_vec.reshape(1, 1, 1, -1), low_band=low_band).item())

    def _decode_attention(self, query, key, value, G):
        B, Hq, _, d = query.shape
        Hkv, Skv = key.shape[1], key.shape[2]
        T = Skv // TILE
        tau = self._tau()
        nc = self.norm_cache
        if Hkv > nc.num_kv_heads or T > nc.max_tiles:
            raise IndexError(f"norm cache ({nc.num_kv_heads} heads x {nc.max_tiles} tiles) is smaller than the "
                             f"context ({Hkv} heads x {T} tiles)")
        if self.score_new_tiles and T > self._prefill_tiles:
            # the tiles completed since the prefill, scored from this call's K
            nc.update_tiles(key[B - 1], self._prefill_tiles, T - self._prefill_tiles, norm_scale=_HOOK_NORM_SCALE)
        # one library call: the Walsh-subspace q norms, their group medians,
        # the gate over the complete tiles (the partial last tile attended)
        # and the decode over the retained tiles
        out, dev = X.hook_decode(query, key, value, nc.cache, G, tau * TILE * d, _LOW_BAND,
                                 stats_out=self.stats.ring_rows(query.device, (B, Hkv, 3)))
        # dev (B, Hkv, 3), written by the gate kernel: evicted complete
        # tiles, the group's q norm and the largest K norm per kv head,
        # reduced over the heads (and clamped at 0) when folded
        stats, gov = self.stats, self.governor

        fold, fold_many = _decode_folds(stats, gov, B, Hkv, T)
        # without a governor, runs of decode calls of one shape fold together
        stats.defer(fold, dev, None if gov is not None else (("decode", B, Hkv, T), fold_many))
        if gov is not None:
            stats.fold()
        return out

    # ------------------------------------------------------------ dense

    def _dense_attention(self, query, key, value, G):
        """Causal attention with nothing gated (perplexity_eval.py:675-689)."""
        key, value = _distinct_kv(query, key, value, G)
        out, _ = X.prefill_attention(query, key, value)
        return out


# plain dict access for the folds, which run inside _Stats.fold (the folding
# accessors would only call it again)
_dget, _dset = dict.__getitem__, dict.__setitem__


def _add(stats, key: str, n) -> None:
    _dset(stats, key, _dget(stats, key) + n)


def _exhaust(stats, max_q: float, max_k: float) -> None:
    """The hallucination-exhaust entries of one batch element (perplexity_eval.py:506-510)."""
    _dget(stats, 'hallucination_scores').append(max_q / (max_k + 1e-10))
    _dget(stats, 'q_search_intensity').append(max_q)
    _dget(stats, 'k_info_density').append(max_k)


def _decode_folds(stats, gov, B: int, Hkv: int, T: int):
    """The folds of a decode call's statistics (B, Hkv, 3): evicted complete
    tiles, the group's q norm and the largest K norm per (batch, kv head)
    (perplexity_eval.py:653-671).  fold(host) folds one call; fold_many(host)
    n calls (n, B, Hkv, 3) at once, entries in call order, batch element
    fastest, with the same float64 values."""

    def fold(host):
        for b in range(B):
            hb = host[b]
            skipped = int(hb[:, 0].sum())
            _exhaust(stats, float(np.maximum(hb[:, 1].max(), 0.0)), float(np.maximum(hb[:, 2].max(), 0.0)))
            _add(stats, 'decode_steps', 1)
            _add(stats, 'decode_tiles_skipped', skipped)
            _add(stats, 'decode_tiles_total', T * Hkv)
            if gov is not None and T > 0:
                gov.report_layer(skipped / (T * Hkv))
        _add(stats, 'layers_processed', 1)

    def fold_many(host):
        mq = np.maximum(host[..., 1].max(axis=2), 0.0).ravel()
        mk = np.maximum(host[..., 2].max(axis=2), 0.0).ravel()
        _dget(stats, 'hallucination_scores').extend((mq / (mk + 1e-10)).tolist())
        _dget(stats, 'q_search_intensity').extend(mq.tolist())
        _dget(stats, 'k_info_density').extend(mk.tolist())
        _add(stats, 'decode_steps', mq.size)
        _add(stats, 'decode_tiles_skipped', int(host[..., 0].sum(axis=2).astype(np.int64).sum()))
        _add(stats, 'decode_tiles_total', T * Hkv * mq.size)
        _add(stats, 'layers_processed', host.shape[0])

    return fold, fold_many


def _distinct_kv(query, key, value, G):
    """k, v with num_kv_heads = num_q_heads / G heads: a k, v already expanded
    to num_q_heads heads by repeat_kv (head j copied to j*G .. j*G + G - 1)
    is reduced to every G-th head."""
    if G > 1 and key.shape[1] == query.shape[1]:
        return key[:, ::G], value[:, ::G]
    return key, value


def patch_model_attention(model, orthocache: OrthoCache_GQA_Attention, min_layer: int = 0):
    """Route the SDPA call of every decoder layer >= min_layer of a
    transformers Llama-style model through `orthocache`
    (perplexity_eval.py:693-741): during the layer's forward,
    torch.nn.functional.scaled_dot_product_attention is replaced by the
    hook (its mask, dropout and scale arguments are ignored, as there: the
    hook is causal with scale 1/sqrt(head_dim))."""
    num_kv_heads = model.config.num_key_value_heads
    num_q_heads = model.config.num_attention_heads
    G = num_q_heads // num_kv_heads
    layers = model.model.layers
    patched = 0
    for idx, layer in enumerate(layers):
        if idx < min_layer:
            continue
        attn = layer.self_attn

        def make(original):
            def patched_forward(*args, **kwargs):
                def intercept(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None,
                              enable_gqa=False):
                    return orthocache.orthocache_attention(query, key, value, num_query_groups=G)

                saved = F.scaled_dot_product_attention
                F.scaled_dot_product_attention = intercept
                try:
                    return original(*args, **kwargs)
                finally:
                    F.scaled_dot_product_attention = saved
            return patched_forward

        attn.forward = make(attn.forward)
        patched += 1
    print(f"  Patched {patched}/{len(layers)} layers (G={G}, layers {min_layer}-{len(layers) - 1})")
    return model
