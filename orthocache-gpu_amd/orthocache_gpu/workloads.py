"""Synthetic decode workloads (used by bench.py and the tests).

Key tiles follow the reference's benchmark recipe in its own band
semantics: a 64-token tile is built in the Walsh domain, K = W64 @ C, so
that its band energies are known by construction
(benchmarks/profile_multihead.py:91-106, profile_fusion.py:164-201):

* smooth tile: rows 1..4 of C ~ N(0,1) (the natural-order "low" band
  [1,8)), plus 0.05*N(0,1) token noise -> E_low ~ 512*d/128, E_high ~ 0.32*d/128,
  zeta ~ 0.02 (retained by the zeta gate, evicted by the CS gate at a tau
  between the clusters);
* noise tile: rows 32..63 of C ~ N(0,1) (the "high" band) -> E_low ~ 0,
  zeta ~ 1e6+ (evicted by the zeta gate, retained by the CS gate).

Each row (sequence x kv head) gets exactly round(noise_frac*T) noise tiles
at random positions (a per-row permutation, as profile_multihead.py:99-102
shuffles tile order per head).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

TILE = 64


def walsh64(device=None, dtype=torch.float32) -> torch.Tensor:
    i = torch.arange(64)
    x = i[:, None] & i[None, :]
    pc = torch.zeros_like(x)
    for b in range(6):
        pc += (x >> b) & 1
    w = (1.0 - 2.0 * (pc % 2).to(torch.float32)) / 8.0
    return w.to(device=device, dtype=dtype)


@dataclass
class KVWorkload:
    keys: torch.Tensor         # (rows, S, d) in the storage dtype
    values: torch.Tensor       # (rows, S, d)
    noise: torch.Tensor        # (rows, T) bool: True = noise tile
    k_scales: Optional[torch.Tensor] = None  # (rows, T) fp32 for fp8 storage
    v_scales: Optional[torch.Tensor] = None


def make_kv(rows: int, seq_len: int, head_dim: int, *, noise_frac: float = 0.5, dtype=torch.bfloat16,
            device="cpu", seed: int = 0, chunk_rows: int = 8, smooth_noise: float = 0.05) -> KVWorkload:
    """Rows of mixed smooth/noise key tiles and N(0,1) values (see module doc).
    dtype float8_e4m3fn stores K and V with one fp32 scale per (row, tile)
    = amax/448 of the bf16 tile."""
    assert seq_len % TILE == 0
    t_count = seq_len // TILE
    g = torch.Generator(device=device).manual_seed(seed)
    w = walsh64(device)
    n_noise = int(round(noise_frac * t_count))
    fp8 = dtype == torch.float8_e4m3fn
    store = torch.bfloat16 if fp8 else dtype
    keys = torch.empty((rows, seq_len, head_dim), dtype=store, device=device)
    values = torch.empty((rows, seq_len, head_dim), dtype=store, device=device)
    noise = torch.zeros((rows, t_count), dtype=torch.bool, device=device)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        nr = r1 - r0
        perm = torch.stack([torch.randperm(t_count, generator=g, device=device) for _ in range(nr)])
        is_noise = perm < n_noise                                   # (nr, T)
        c = torch.zeros((nr, t_count, TILE, head_dim), device=device)
        c[:, :, 1:5] = torch.randn((nr, t_count, 4, head_dim), generator=g, device=device)
        hi = torch.randn((nr, t_count, 32, head_dim), generator=g, device=device)
        c[:, :, 32:64] = hi * is_noise[..., None, None]
        c[:, :, 1:5] *= (~is_noise)[..., None, None]
        k = torch.matmul(w, c)                                      # (nr, T, 64, d)
        k += smooth_noise * torch.randn(k.shape, generator=g, device=device) * (~is_noise)[..., None, None]
        keys[r0:r1] = k.reshape(nr, seq_len, head_dim).to(store)
        values[r0:r1] = torch.randn((nr, seq_len, head_dim), generator=g, device=device).to(store)
        noise[r0:r1] = is_noise
        del c, k, hi
    if not fp8:
        return KVWorkload(keys, values, noise)
    kq, ks = quantize_fp8_tiles(keys)
    vq, vs = quantize_fp8_tiles(values)
    return KVWorkload(kq, vq, noise, ks, vs)


def make_kv_literal(rows: int, seq_len: int, head_dim: int, *, dtype=torch.float32, seed: int = 0):
    """The config text read literally, with the Walsh rows along head_dim:
    every token's key is a combination of natural-order rows of H_head_dim
    with its own N(0, 1) coefficients -- rows 1..4 (plus 0.05 N(0, 1)) in
    half the tiles, rows head_dim/2 .. head_dim-1 in the other half.  Along
    the tokens every tile is then white noise, so the 64-point token-axis
    zeta of every tile centres on 32/7 (about 4.58) whatever its label, and
    zeta_max = 5 evicts a label-independent share (about 12% of the "noise"
    and 40% of the "smooth" tiles at head_dim 128)."""
    g = torch.Generator().manual_seed(seed)
    i = torch.arange(head_dim)
    pc = torch.zeros((head_dim, head_dim), dtype=torch.int64)
    x = i[:, None] & i[None, :]
    while bool(x.any()):
        pc += x & 1
        x = x >> 1
    wd = (1.0 - 2.0 * (pc % 2).float()) / head_dim ** 0.5    # H_d / sqrt(d), rows = sequency basis
    t_count = seq_len // TILE
    coef = torch.zeros((rows, t_count, TILE, head_dim))
    noise = torch.rand((rows, t_count), generator=g) < 0.5
    low = torch.randn((rows, t_count, TILE, 4), generator=g)
    high = torch.randn((rows, t_count, TILE, head_dim // 2), generator=g)
    coef[..., 1:5] = low * (~noise)[..., None, None]
    coef[..., head_dim // 2:] = high * noise[..., None, None]
    k = coef @ wd
    k += 0.05 * torch.randn(k.shape, generator=g) * (~noise)[..., None, None]
    return k.reshape(rows, seq_len, head_dim).to(dtype), noise


def quantize_fp8_tiles(x: torch.Tensor):
    """Per-(row, 64-token tile) scale = amax/448 (1 for an all-zero tile);
    returns (e4m3fn tensor, (rows, T) float32 scales)."""
    rows, s_len, d = x.shape
    t = x.float().view(rows, s_len // TILE, TILE, d)
    amax = t.abs().amax(dim=(2, 3))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (t / scale[..., None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(rows, s_len, d), scale.contiguous()


def make_q(rows: int, G: int, head_dim: int, *, dtype=torch.bfloat16, device="cpu", seed: int = 1,
           low_band_heads: int = 0) -> torch.Tensor:
    """(rows*G, d) N(0,1) queries.  The first `low_band_heads` of each group
    are projected onto natural rows [0, 8) of the head_dim Walsh basis
    (config 2's "zero high-band energy" heads)."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn((rows, G, head_dim), generator=g, device=device)
    if low_band_heads:
        n = head_dim
        i = torch.arange(n, device=device)
        x = i[:, None] & i[None, :]
        pc = torch.zeros_like(x)
        for b in range(int(math.log2(n))):
            pc += (x >> b) & 1
        h = (1.0 - 2.0 * (pc % 2).float()) / math.sqrt(n)
        coeff = q[:, :low_band_heads] @ h.T
        coeff[..., 8:] = 0
        q[:, :low_band_heads] = coeff @ h
    return q.reshape(rows * G, head_dim).to(dtype)


def calibrate_tau(e_high: torch.Tensor, q: torch.Tensor, G: int, live: Optional[torch.Tensor] = None) -> float:
    """A CS threshold halfway (geometrically) between the largest bound of a
    row's smooth tiles and the smallest of its noise tiles, pooled over rows
    (the reference calibrates zeta_max from sorted scores,
    profile_multihead.py:108-118).  `live` (rows, T) bool: the tiles inside
    each row's length (rows of different lengths)."""
    rows = e_high.shape[0]
    qn = q.float().view(rows, G, -1).norm(dim=2).amax(dim=1)
    cs = qn[:, None] * e_high.float().sqrt()
    cs = cs.flatten() if live is None else cs[live]
    # split the two clusters at the largest multiplicative gap
    v = cs.sort().values.clamp(min=1e-30)
    gaps = v[1:] / v[:-1]
    k = int(gaps.argmax())
    return float(math.sqrt(float(v[k]) * float(v[k + 1])))


def paged_pool(keys: torch.Tensor, values: torch.Tensor, num_kv_heads: int, block_size: int,
               lengths, *, seed: int = 0, extra_blocks: int = 3):
    """Scatter (B*Hkv, S, d) rows into a shuffled physical page pool.

    Returns (k_cache, v_cache, block_tables int32 (B, max_blocks)); sequence
    b uses ceil(lengths[b]/block_size) pages, unused table entries are -1."""
    rows, s_len, d = keys.shape
    b_count = rows // num_kv_heads
    lens = [int(x) for x in lengths]
    need = [-(-n // block_size) for n in lens]
    max_blocks = -(-s_len // block_size)
    total = sum(need) + extra_blocks
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(total, generator=g)
    bt = torch.full((b_count, max_blocks), -1, dtype=torch.int32)
    k_cache = torch.zeros((total, num_kv_heads, block_size, d), dtype=keys.dtype, device=keys.device)
    v_cache = torch.zeros(k_cache.shape, dtype=values.dtype, device=values.device)
    pos = 0
    kr = keys.view(b_count, num_kv_heads, s_len, d)
    vr = values.view(b_count, num_kv_heads, s_len, d)
    for b in range(b_count):
        ids = perm[pos:pos + need[b]]
        pos += need[b]
        bt[b, :need[b]] = ids.to(torch.int32)
        n_full = need[b] * block_size
        kb = torch.zeros((num_kv_heads, n_full, d), dtype=keys.dtype, device=keys.device)
        vb = torch.zeros(kb.shape, dtype=values.dtype, device=values.device)
        take = min(n_full, s_len)
        kb[:, :take] = kr[b, :, :take]
        vb[:, :take] = vr[b, :, :take]
        idx = ids.to(keys.device)
        k_cache[idx] = kb.view(num_kv_heads, need[b], block_size, d).permute(1, 0, 2, 3)
        v_cache[idx] = vb.view(num_kv_heads, need[b], block_size, d).permute(1, 0, 2, 3)
    return k_cache, v_cache, bt.to(keys.device)
