"""Eviction regimes of the compact pipeline (the API of src/orthocache_gpu/
perfect_eviction.py in the reference).

An evicted block's largest possible logit is its ceiling
beta = max_h ||q_h||max * sqrt(E_h) / sqrt(d) (Cauchy-Schwarz over the
block's keys, E_h their energy).  When the largest retained logit z lies at
least the accumulator's exp-underflow distance above beta, every exp of the
block's logits rounds to zero, so evicting it changes nothing ("perfect");
otherwise its weight is only bounded ("statistical").

The whole classification runs in one HIP launch, oc_block_regimes, on the
query norms of oc_row_norms; this module only shapes arguments and results.
Tensors must live on the GPU (there is no CPU path).
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

import torch

from . import _launch as X

# exp(x) of a float32 accumulator is exactly 0 below x = -88.72, of a
# bfloat16 one below -87.34 (perfect_eviction.py:47-53); kept by value
FLOAT32_UNDERFLOW_THRESHOLD: float = 88.72
BFLOAT16_UNDERFLOW_THRESHOLD: float = 87.34

_UNDERFLOW = {"float32": FLOAT32_UNDERFLOW_THRESHOLD, "bfloat16": BFLOAT16_UNDERFLOW_THRESHOLD}


def _underflow(accumulator_dtype: str) -> float:
    # any other name means a float32 accumulator, as in the reference
    return _UNDERFLOW.get(accumulator_dtype, FLOAT32_UNDERFLOW_THRESHOLD)


class EvictionRegime(Enum):
    """Regime codes (perfect_eviction.py:56-61)."""
    RETAIN = "retain"
    PERFECT_EVICTION = "perfect"
    STATISTICAL_EVICTION = "statistical"


@dataclass
class EvictionMetadata:
    """Per-block result of classify_eviction (perfect_eviction.py:64-72);
    regime holds 0 (retained), 1 (perfect) or 2 (statistical)."""
    regime: torch.Tensor
    beta: torch.Tensor
    logit_gap: torch.Tensor
    num_perfect: int
    num_statistical: int
    num_retained: int
    underflow_threshold: float


def compute_block_beta(q: torch.Tensor, block_energies: torch.Tensor, head_dim: int) -> torch.Tensor:
    """(num_blocks, num_heads) logit ceilings ||q_h||max sqrt(E) / sqrt(head_dim)
    for q (q_len, num_heads, d) (perfect_eviction.py:75-104)."""
    nb = block_energies.shape[0]
    keep_all = torch.ones((nb,), dtype=torch.uint8, device=block_energies.device)
    *_, full, _ = X.block_regimes(q, block_energies, head_dim, 0.0, keep_all, FLOAT32_UNDERFLOW_THRESHOLD,
                                  want_full=True)
    return full


def classify_eviction(q: torch.Tensor, block_energies: torch.Tensor, z_max, block_mask: torch.Tensor, head_dim: int,
                      accumulator_dtype: str = "float32") -> EvictionMetadata:
    """Regime of every block (perfect_eviction.py:107-186).  block_mask (True =
    retained) is per block or per (block, head), a block counting as retained
    when any head keeps it; z_max is a number or a tensor whose largest
    element is taken.  The counts are read back to the host."""
    thr = _underflow(accumulator_dtype)
    regime, beta, gap, _, counts = X.block_regimes(q, block_energies, head_dim, z_max, block_mask, thr)
    n_perfect, n_stat, n_kept = counts.tolist()
    return EvictionMetadata(regime=regime, beta=beta, logit_gap=gap, num_perfect=n_perfect,
                            num_statistical=n_stat, num_retained=n_kept, underflow_threshold=thr)


def perfect_eviction_check(z_max: float, beta: float, accumulator_dtype: str = "float32") -> bool:
    """Whether one block with ceiling beta is perfectly evicted under the
    largest retained logit z_max (perfect_eviction.py:189-212)."""
    return z_max - beta >= _underflow(accumulator_dtype)
