"""OrthoCache spectral-gated decode attention for AMD Instinct MI355X.

Drop-in for the decode path of the reference package `orthocache_gpu`:
the fused FWHT + zeta / Cauchy-Schwarz gate + split-K flash-decode entry
points keep their module paths, signatures and metadata, and run on
hand-written HIP kernels for gfx950 (liborthocache_hip.so, C ABI in
include/orthocache_hip.h).  Inputs must be GPU tensors; there is no CPU
fallback.
"""

__version__ = "0.1.0"

from .pipeline import (  # noqa: F401
    orthocache_forward,
    CROSSOVER_SEQ_LEN,
    GPUProfile,
    get_hardware_profile,
    get_crossover_threshold,
    BypassFlag,
    TelemetryLevel,
    format_bypass_reason,
)
from .triton_kernels.fwht_fused_prototype import (  # noqa: F401
    triton_fwht_eviction,
    generate_walsh_matrix,
    score_tiles,
    fwht_tiles,
    TileScores,
)
from .triton_kernels.fused_eviction import (  # noqa: F401
    fused_orthocache_attention,
    fused_orthocache_attention_v2,
)
from .triton_kernels.gqa_eviction import fused_orthocache_attention_v3_gqa  # noqa: F401
from .triton_kernels.paged_eviction import (  # noqa: F401
    fused_orthocache_attention_paged,
    score_paged_tiles,
)

__all__ = [
    "__version__",
    "orthocache_forward",
    "CROSSOVER_SEQ_LEN",
    "GPUProfile",
    "get_hardware_profile",
    "get_crossover_threshold",
    "BypassFlag",
    "TelemetryLevel",
    "format_bypass_reason",
    "triton_fwht_eviction",
    "generate_walsh_matrix",
    "score_tiles",
    "fwht_tiles",
    "TileScores",
    "fused_orthocache_attention",
    "fused_orthocache_attention_v2",
    "fused_orthocache_attention_v3_gqa",
    "fused_orthocache_attention_paged",
    "score_paged_tiles",
]
