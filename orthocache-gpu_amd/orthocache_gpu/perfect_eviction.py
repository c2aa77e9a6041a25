"""Eviction regimes of the compact pipeline (src/orthocache_gpu/
perfect_eviction.py of the reference): an evicted block whose logit
ceiling beta lies at least the float32 exp-underflow distance below the
largest retained logit contributes exactly zero to a float32 softmax
("perfect" eviction); the others are "statistical".  These are per-block
scalars over (num_blocks, num_heads) tensors the spectra kernel produced.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum

import torch

FLOAT32_UNDERFLOW_THRESHOLD: float = 88.72
BFLOAT16_UNDERFLOW_THRESHOLD: float = 87.34


class EvictionRegime(Enum):
    RETAIN = "retain"
    PERFECT_EVICTION = "perfect"
    STATISTICAL_EVICTION = "statistical"


@dataclass
class EvictionMetadata:
    regime: torch.Tensor        # (num_blocks,) int32: 0 retain, 1 perfect, 2 statistical
    beta: torch.Tensor          # (num_blocks,) logit ceiling, max over heads
    logit_gap: torch.Tensor     # (num_blocks,) z_max - beta
    num_perfect: int
    num_statistical: int
    num_retained: int
    underflow_threshold: float


def compute_block_beta(q: torch.Tensor, block_energies: torch.Tensor, head_dim: int) -> torch.Tensor:
    """beta = max_s ||q_s|| sqrt(E) / sqrt(head_dim), (num_blocks, num_heads)
    (perfect_eviction.py:75-104)."""
    q_norm_max = torch.linalg.vector_norm(q.float(), dim=-1).amax(dim=0)
    return (q_norm_max[None, :] * torch.sqrt(block_energies.float().clamp(min=0))) / math.sqrt(head_dim)


def classify_eviction(q: torch.Tensor, block_energies: torch.Tensor, z_max, block_mask: torch.Tensor, head_dim: int,
                      accumulator_dtype: str = "float32") -> EvictionMetadata:
    """Per-block regime of the evicted blocks (perfect_eviction.py:107-186)."""
    threshold = BFLOAT16_UNDERFLOW_THRESHOLD if accumulator_dtype == "bfloat16" else FLOAT32_UNDERFLOW_THRESHOLD
    beta_max = compute_block_beta(q, block_energies, head_dim).amax(dim=-1)
    if isinstance(z_max, torch.Tensor) and z_max.ndim > 0:
        z = float(z_max.max().item())
    else:
        z = float(z_max)
    gap = z - beta_max
    unified = block_mask.any(dim=-1) if block_mask.ndim > 1 else block_mask
    evicted = ~unified
    perfect = evicted & (gap >= threshold)
    statistical = evicted & (gap < threshold)
    regime = torch.zeros(unified.shape[0], dtype=torch.int32, device=q.device)
    regime[perfect] = 1
    regime[statistical] = 2
    counts = torch.stack([perfect.sum(), statistical.sum(), unified.sum()]).tolist()
    return EvictionMetadata(regime=regime, beta=beta_max, logit_gap=gap, num_perfect=int(counts[0]),
                            num_statistical=int(counts[1]), num_retained=int(counts[2]),
                            underflow_threshold=threshold)


def perfect_eviction_check(z_max: float, beta: float, accumulator_dtype: str = "float32") -> bool:
    """z_max - beta >= the accumulator's underflow threshold (perfect_eviction.py:189-212)."""
    threshold = BFLOAT16_UNDERFLOW_THRESHOLD if accumulator_dtype == "bfloat16" else FLOAT32_UNDERFLOW_THRESHOLD
    return (z_max - beta) >= threshold
