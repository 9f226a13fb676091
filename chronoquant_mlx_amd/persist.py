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

Opt-in dense residuals (save_prompt_cache(..., dense=True)): a component
whose residual codes have 2 or 3 bits stores them in the file as a bit stream
of that width instead of the reference's INT4 lanes (3-bit: 48 instead of 64
bytes per 128-dim row).  Such a file is this library's format only: the
reference cannot read it.  The stream is the same one a dense_residuals
cache holds in HBM (its rows are the stream padded to whole words), so such
a cache saves its rows as they are; a cache loaded from the file takes the
layout its own dense_residuals setting asks for.
"""
from __future__ import annotations

import json

import torch

from .cache import ChronoQuantCache
from .host import KVCache

_FORMAT = "chronoquant_mlx_amd.prompt_cache.v1"
_CHUNK_ROWS = 1 << 16  # rows packed / unpacked at a time (bounds the bit expansion)


def _u32_to_i64(words: torch.Tensor) -> torch.Tensor:
    return words.view(torch.int32).to(torch.int64) & 0xFFFFFFFF


def dense_pack(words: torch.Tensor, head_dim: int, bits: int) -> torch.Tensor:
    """INT4-lane rows [..., W] (uint32; nibble i of word w = code(8w + i) + 8,
    nibbles of dims >= head_dim 0) -> the codes of dims < head_dim as a
    little-endian stream of `bits`-bit fields holding code + 2^(bits-1):
    field d occupies stream bits [bits*d, bits*d + bits).  uint8 [...,
    ceil(head_dim * bits / 8)].  Raises if a code is out of the bits' range."""
    if bits not in (2, 3):
        raise ValueError("dense residuals are 2 or 3 bits")
    W, D = words.shape[-1], head_dim
    lead = words.shape[:-1]
    nbytes = (D * bits + 7) // 8
    flat = words.reshape(-1, W)
    out = torch.empty(flat.shape[0], nbytes, dtype=torch.uint8, device=words.device)
    base = 8 - (1 << (bits - 1))
    sh4 = 4 * torch.arange(8, device=words.device)
    shb = torch.arange(bits, device=words.device)
    sh8 = torch.arange(8, device=words.device)
    for r0 in range(0, flat.shape[0], _CHUNK_ROWS):
        w = _u32_to_i64(flat[r0:r0 + _CHUNK_ROWS])
        nib = ((w[:, :, None] >> sh4) & 0xF).reshape(w.shape[0], W * 8)[:, :D]
        vals = nib - base
        if bool(((vals < 0) | (vals >= (1 << bits))).any()):
            raise ValueError(f"a code does not fit {bits} bits")
        stream = ((vals[:, :, None] >> shb) & 1).reshape(w.shape[0], D * bits)
        stream = torch.nn.functional.pad(stream, (0, nbytes * 8 - D * bits))
        out[r0:r0 + _CHUNK_ROWS] = ((stream.reshape(-1, nbytes, 8) << sh8).sum(-1)).to(torch.uint8)
    return out.reshape(*lead, nbytes)


def dense_unpack(stream: torch.Tensor, head_dim: int, bits: int) -> torch.Tensor:
    """Inverse of dense_pack: uint8 [..., nbytes] -> uint32 INT4-lane rows
    [..., ceil(head_dim / 8)] (pad nibbles 0)."""
    D = head_dim
    W = (D + 7) // 8
    nbytes = stream.shape[-1]
    if nbytes != (D * bits + 7) // 8:
        raise ValueError("dense stream size does not match head_dim and bits")
    lead = stream.shape[:-1]
    flat = stream.reshape(-1, nbytes)
    out = torch.empty(flat.shape[0], W, dtype=torch.int32, device=stream.device)
    base = 8 - (1 << (bits - 1))
    sh8 = torch.arange(8, device=stream.device)
    shb = torch.arange(bits, device=stream.device)
    sh4 = 4 * torch.arange(8, device=stream.device)
    for r0 in range(0, flat.shape[0], _CHUNK_ROWS):
        b = flat[r0:r0 + _CHUNK_ROWS].to(torch.int64)
        bitv = ((b[:, :, None] >> sh8) & 1).reshape(b.shape[0], nbytes * 8)[:, :D * bits]
        vals = (bitv.reshape(-1, D, bits) << shb).sum(-1)
        nib = torch.nn.functional.pad(vals + base, (0, W * 8 - D))
        word = (nib.reshape(-1, W, 8) << sh4).sum(-1)  # < 2^32
        out[r0:r0 + _CHUNK_ROWS] = (word - ((word >> 31) << 32)).to(torch.int32)
    return out.view(torch.uint32).reshape(*lead, W)


def _dense_bits(c) -> dict:
    """State index -> residual bits of each 2- or 3-bit packed component."""
    bits = {2: int(c.delta_bits_k), 4: int(c._get_codec_for_v().delta_bits)}
    return {i: b for i, b in bits.items() if b in (2, 3)}


_PARAMS = ("stride_k", "stride_v", "delta_bits_k", "delta_bits_v", "dead_zone_k", "dead_zone_v",
           "use_fused", "layer_idx", "dense_residuals")


def _layer_info(c) -> dict:
    if isinstance(c, ChronoQuantCache):
        return {"class": "ChronoQuantCache", "params": {p: getattr(c, p) for p in _PARAMS},
                "per_layer_v_bits": c.per_layer_v_bits, "meta_state": c.meta_state}
    if isinstance(c, KVCache):
        return {"class": "KVCache", "meta_state": c.meta_state}
    raise TypeError(f"cannot save a cache of type {type(c).__name__}")


def save_prompt_cache(file_name: str, cache: list, metadata: dict | None = None,
                      dense: bool = False) -> None:
    """Write every layer's state (device tensors are copied to the host).
    dense: store 2- and 3-bit residual codes at their width (opt-in; see the
    module docstring)."""
    from safetensors.torch import save_file
    tensors = {}
    info = [_layer_info(c) for c in cache]
    for i, c in enumerate(cache):
        state = c.state
        is_cq = isinstance(c, ChronoQuantCache) and bool(state)
        packed = _dense_bits(c) if dense and is_cq else {}
        # components whose rows are dense in HBM (dense_residuals caches)
        in_hbm = {j: b for j, b in (_dense_bits(c) if is_cq and c.dense_residuals else {}).items()}
        for j, t in enumerate(state):
            t = t.detach().contiguous()
            if j in in_hbm:
                nbytes = (c.head_dim * in_hbm[j] + 7) // 8
                stream = t.view(torch.uint8)[..., :nbytes]  # the rows are this stream
                t = stream if j in packed else dense_unpack(stream, c.head_dim, in_hbm[j])
            elif j in packed:
                t = dense_pack(t, c.head_dim, packed[j])
            tensors[f"{i}.{j}"] = t.contiguous().cpu()
        if packed:
            info[i]["dense"] = {"head_dim": int(c.head_dim),
                                "bits": {str(j): b for j, b in packed.items()}}
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
        dense = layer.get("dense")
        if dense:
            for j, b in dense["bits"].items():
                state[int(j)] = dense_unpack(state[int(j)], dense["head_dim"], b)
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
