"""Monkey-patch of the host framework's SDPA symbol + cache factories.

Mirrors the reference patch.py (gauravsaini/chronoquant_mlx, patch.py:1-104)
against the PyTorch host surface in chronoquant_mlx_amd.host instead of
mlx_lm.models.base.
"""
from __future__ import annotations

import sys

from . import host as _base
from .attention import chronoquant_sdpa
from .cache import ChronoQuantCache

_original_sdpa = _base.scaled_dot_product_attention
_patched = False

# Modules whose `scaled_dot_product_attention` binding apply() rebinds (the
# reference walks every "mlx_lm.models.*" module, patch.py:28-30).
MODEL_MODULE_PREFIXES = ["chronoquant_mlx_amd.models."]


def register_model_module(prefix: str) -> None:
    """Make apply() rebind the SDPA symbol in modules named `prefix`*."""
    if prefix not in MODEL_MODULE_PREFIXES:
        MODEL_MODULE_PREFIXES.append(prefix)
    if _patched:
        _rebind(_patched_sdpa)


def _patched_sdpa(queries, keys, values, cache, scale, mask, **kwargs):
    """patch.py:12-15: ChronoQuant caches go to chronoquant_sdpa."""
    if isinstance(cache, ChronoQuantCache):
        return chronoquant_sdpa(queries, keys, values, cache, scale, mask)
    return _original_sdpa(queries, keys, values, cache, scale, mask, **kwargs)


def _rebind(fn) -> None:
    for name, module in list(sys.modules.items()):
        if module is None:
            continue
        if any(name.startswith(p) for p in MODEL_MODULE_PREFIXES) and hasattr(
                module, "scaled_dot_product_attention"):
            module.scaled_dot_product_attention = fn


def apply_patch():
    """Route the host framework's attention symbol to chronoquant_sdpa for
    ChronoQuant caches (patch.py:18-33); calling it again changes nothing."""
    global _patched
    if _patched:
        return
    _base.scaled_dot_product_attention = _patched_sdpa
    _rebind(_patched_sdpa)
    _patched = True
    print("chronoquant_mlx_amd: scaled_dot_product_attention now sends ChronoQuant caches "
          "to the gfx950 kernels")


def apply():
    apply_patch()


def revert():
    """patch.py:40-43 (also restores the rebound model modules)."""
    global _patched
    _base.scaled_dot_product_attention = _original_sdpa
    _rebind(_original_sdpa)
    _patched = False


def create_chronoquant_caches(
    model,
    stride_k: int = 32,
    stride_v: int = 8,
    delta_bits_k: int = 4,
    delta_bits_v: int = 4,
    dead_zone_k: float = 0.0,
    dead_zone_v: float = 0.05,
    use_fused: bool = True,
    per_layer_v_bits: list = None,
    dense_residuals: bool = False,
):
    """Replace every plain KVCache slot of the model's prompt cache with a
    ChronoQuantCache of these codec settings (patch.py:46-78).

    per_layer_v_bits: value residual width by layer index (layers past the
    end of the list take its last entry); None uses delta_bits_v everywhere.
    dense_residuals (no reference counterpart, opt-in): 2- and 3-bit
    components keep their codes at their own width in HBM.
    """
    caches = _base.make_prompt_cache(model)
    for index in range(len(caches)):
        if isinstance(caches[index], _base.KVCache):
            v_bits = (per_layer_v_bits[index]
                      if per_layer_v_bits and index < len(per_layer_v_bits) else delta_bits_v)
            caches[index] = ChronoQuantCache(
                stride_k=stride_k,
                stride_v=stride_v,
                delta_bits_k=delta_bits_k,
                delta_bits_v=v_bits,
                dead_zone_k=dead_zone_k,
                dead_zone_v=dead_zone_v,
                use_fused=use_fused,
                per_layer_v_bits=per_layer_v_bits,
                dense_residuals=dense_residuals,
            )
            caches[index].layer_idx = index  # selects its entry of per_layer_v_bits
    return caches


FULL_THROTTLE_V3_CONFIG = {  # patch.py:81-88
    "stride_k": 64,
    "stride_v": 32,
    "delta_bits_k": 4,
    "delta_bits_v": 3,
    "dead_zone_k": 0.0,
    "dead_zone_v": 0.05,
}


def create_full_throttle_caches(model, use_fused: bool = True, dense_residuals: bool = False):
    """Create the Full-Throttle V3 cache preset (patch.py:91-104).

    3-bit V residuals occupy INT4 lanes, as in the reference, unless
    dense_residuals (this library's opt-in) stores them as 48-byte rows.
    """
    return create_chronoquant_caches(model, use_fused=use_fused, dense_residuals=dense_residuals,
                                     **FULL_THROTTLE_V3_CONFIG)
