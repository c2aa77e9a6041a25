"""512-token block spectra of the compact pipeline (src/orthocache_gpu/
spectral_energy.py and fwht.py of the reference).

The reference transforms every (512-token block, head) with fwht_512 (a
normalised natural-order Walsh-Hadamard transform along tokens) and sums
squared coefficients per sequency band; here one oc_block_spectra launch
reads each block once and returns every band energy, the spectral decay
ratio, the spatial energy, the block mean and the query-aware bounds.
Arithmetic is float32 whatever the key dtype (the reference's butterflies
run in the keys' dtype, so 16-bit keys agree to that dtype's rounding).
The band boundaries are the reference's defaults; other bands raise
NotImplementedError.
"""

from __future__ import annotations

import torch

from . import _launch as X

BAND_DC = 0
BAND_LOW = (1, 64)
BAND_MID = (64, 256)
BAND_HIGH = (256, 512)


def _check(keys: torch.Tensor, block_size: int) -> None:
    if block_size != X.SPECTRA_BLOCK:
        raise NotImplementedError(f"block_size {block_size}: the transform is 512-point (fwht_512)")
    if keys.dim() != 3:
        raise ValueError(f"keys must be (seq_len, num_heads, head_dim), got {tuple(keys.shape)}")
    if keys.shape[0] % block_size:
        # the reference's keys.reshape(num_blocks, block_size, ...) fails the same way
        raise RuntimeError(f"shape '{[keys.shape[0] // block_size, block_size, *keys.shape[1:]]}' is invalid for "
                           f"input of size {keys.numel()}")


def _bands_default(band_low, band_mid, band_high) -> None:
    if tuple(band_low) != BAND_LOW or tuple(band_mid) != BAND_MID or tuple(band_high) != BAND_HIGH:
        raise NotImplementedError("only the default sequency bands [1,64), [64,256), [256,512) are computed")


def compute_block_energy(keys: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """sum over a block's tokens and head_dim of k^2, (num_blocks, num_heads)
    float32 (spectral_energy.py:20-34)."""
    _check(keys, block_size)
    return X.block_spectra(keys)["energy"]


def compute_spectral_bands(keys: torch.Tensor, block_size: int = 512, band_low: tuple = BAND_LOW,
                           band_mid: tuple = BAND_MID, band_high: tuple = BAND_HIGH) -> tuple:
    """(dc_component (num_blocks, num_heads, head_dim), low, mid, high energies
    (num_blocks, num_heads)) of the normalised 512-point transform
    (spectral_energy.py:68-105)."""
    _check(keys, block_size)
    _bands_default(band_low, band_mid, band_high)
    s = X.block_spectra(keys, want_mean=True)
    dc = s["block_mean"] * (float(block_size) ** 0.5)  # X[0] = sum_t k_t / sqrt(512)
    return dc, s["e_low"], s["e_mid"], s["e_high"]


def compute_spectral_decay_ratio(keys: torch.Tensor, block_size: int = 512, band_low: tuple = BAND_LOW,
                                 band_high: tuple = BAND_HIGH) -> torch.Tensor:
    """zeta = E_high / (E_low + 1e-6) per (block, head) (spectral_energy.py:108-137)."""
    _check(keys, block_size)
    _bands_default(band_low, (band_low[1], band_high[0]), band_high)
    return X.block_spectra(keys)["zeta"]


def compute_query_aware_bounds(q: torch.Tensor, keys: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """(q . block_mean + ||q|| sqrt(E_ac)) / sqrt(head_dim), (seq_len_q,
    num_blocks, num_heads) (spectral_energy.py:140-176)."""
    _check(keys, block_size)
    return X.block_spectra(keys, q, want_bounds=True)["bounds"]


def compute_query_aware_mask(q: torch.Tensor, keys: torch.Tensor, tau: float, block_size: int = 512) -> torch.Tensor:
    """max over queries of the bound >= tau, (num_blocks, num_heads) bool
    (spectral_energy.py:179-195)."""
    _check(keys, block_size)
    return X.block_spectra(keys, q)["max_bound"] >= tau


def compute_multiband_mask(q: torch.Tensor, keys: torch.Tensor, tau: float, zeta_max: float,
                           block_size: int = 512) -> torch.Tensor:
    """Retained iff max bound >= tau and zeta <= zeta_max, (num_blocks,
    num_heads) bool (spectral_energy.py:198-233); one spectra pass."""
    _check(keys, block_size)
    s = X.block_spectra(keys, q)
    return (s["max_bound"] >= tau) & (s["zeta"] <= zeta_max)


def generate_threshold_mask(energies: torch.Tensor, epsilon: float) -> torch.Tensor:
    """energies >= epsilon (spectral_energy.py:236-238)."""
    return energies >= epsilon
