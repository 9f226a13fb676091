"""ChronoQuant KV-cache codec and fused dequant-attention for MI355X (gfx950).

Drop-in counterpart of the reference package's public surface
(gauravsaini/chronoquant_mlx __init__.py:3-21) on PyTorch-ROCm, backed by
the HIP kernels of libchronoquant.so (C ABI: include/chronoquant.h).
"""
from .cache import ChronoQuantCache
from .patch import (
    FULL_THROTTLE_V3_CONFIG,
    apply,
    apply_patch,
    create_chronoquant_caches,
    create_full_throttle_caches,
    revert,
)
from .attention import chronoquant_sdpa
from .persist import load_prompt_cache, save_prompt_cache

__all__ = [
    "ChronoQuantCache",
    "FULL_THROTTLE_V3_CONFIG",
    "apply",
    "apply_patch",
    "create_chronoquant_caches",
    "create_full_throttle_caches",
    "chronoquant_sdpa",
    "revert",
    # prompt-cache files (mlx_lm's save_prompt_cache / load_prompt_cache)
    "save_prompt_cache",
    "load_prompt_cache",
]
