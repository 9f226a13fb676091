"""Prompt-cache files: the counterpart of mlx_lm's save_prompt_cache /
load_prompt_cache for lists of ChronoQuantCache / KVCache layers.

The reference persists a cache through its `state` list (cache.py:220-255),
which mlx_lm writes to one safetensors file under keys "{layer}.{index}".
This module keeps that layout: layer i's state tensors are "i.0", "i.1", ...
in the reference order (keyframes_k, keyframes_v, packed_k, scales_k,
packed_v, scales_v for ChronoQuantCache; keys, values for KVCache).  The
reference's meta_state is empty, so the codec parameters a cache needs to
interpret its tensors (strides, residual bits, dead zones) are stored in the
file's metadata beside the layer's class name.

    save_prompt_cache("prompt.safetensors", caches, {"model": "..."})
    caches = load_prompt_cache("prompt.safetensors")
"""
from __future__ import annotations

import json

import torch

from .cache import ChronoQuantCache
from .host import KVCache

_FORMAT = "chronoquant_mlx_amd.prompt_cache.v1"
_PARAMS = ("stride_k", "stride_v", "delta_bits_k", "delta_bits_v", "dead_zone_k", "dead_zone_v",
           "use_fused", "layer_idx")


def _layer_info(c) -> dict:
    if isinstance(c, ChronoQuantCache):
        return {"class": "ChronoQuantCache", "params": {p: getattr(c, p) for p in _PARAMS},
                "per_layer_v_bits": c.per_layer_v_bits, "meta_state": c.meta_state}
    if isinstance(c, KVCache):
        return {"class": "KVCache", "meta_state": c.meta_state}
    raise TypeError(f"cannot save a cache of type {type(c).__name__}")


def save_prompt_cache(file_name: str, cache: list, metadata: dict | None = None) -> None:
    """Write every layer's state (device tensors are copied to the host)."""
    from safetensors.torch import save_file
    tensors = {}
    for i, c in enumerate(cache):
        for j, t in enumerate(c.state):
            tensors[f"{i}.{j}"] = t.detach().contiguous().cpu()
    info = [_layer_info(c) for c in cache]
    meta = {"format": _FORMAT, "layers": json.dumps(info),
            "n_state": json.dumps([len(c.state) for c in cache]),
            "metadata": json.dumps(metadata or {})}
    save_file(tensors, file_name, metadata=meta)


def load_prompt_cache(file_name: str, return_metadata: bool = False, device: str = "cuda"):
    """Rebuild the list of caches (on `device`) written by save_prompt_cache."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    with safe_open(file_name, "pt") as f:
        meta = f.metadata() or {}
    if meta.get("format") != _FORMAT:
        raise ValueError(f"{file_name} is not a {_FORMAT} file")
    tensors = load_file(file_name, device=device)
    info = json.loads(meta["layers"])
    n_state = json.loads(meta["n_state"])
    caches = []
    for i, (layer, n) in enumerate(zip(info, n_state)):
        state = [tensors[f"{i}.{j}"] for j in range(n)]
        if layer["class"] == "ChronoQuantCache":
            c = ChronoQuantCache(**layer["params"], per_layer_v_bits=layer.get("per_layer_v_bits"))
        elif layer["class"] == "KVCache":
            c = KVCache()
        else:
            raise ValueError(f"unknown cache class {layer['class']}")
        c.state = state
        c.meta_state = layer.get("meta_state", "")
        caches.append(c)
    if return_metadata:
        return caches, json.loads(meta.get("metadata", "{}"))
    return caches
