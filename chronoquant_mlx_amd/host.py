"""The PyTorch host-framework surface the ChronoQuant patch plugs into.

The reference patches mlx_lm (mlx_lm.models.base.scaled_dot_product_attention
and the same symbol in every loaded mlx_lm.models.* module, patch.py:18-33)
and converts mlx_lm KVCache slots (patch.py:61-65).  This module is the
PyTorch counterpart of those three mlx_lm pieces:

* scaled_dot_product_attention(queries, keys, values, cache, scale, mask,
  **kwargs) — the symbol attention modules call after update_and_fetch;
* KVCache — a plain fp16 cache with the same protocol as ChronoQuantCache;
* make_prompt_cache(model) — one KVCache per attention layer.

Any PyTorch attention module that calls scaled_dot_product_attention from a
module registered with patch.register_model_module() is re-routed by apply().
"""
from __future__ import annotations

import torch


def scaled_dot_product_attention(queries, keys, values, cache, scale: float, mask=None,
                                 **kwargs):
    """Dense GQA attention.  queries [B, nq, L, D]; keys/values [B, nkv, S, D]."""
    B, nq, L, D = queries.shape
    nkv = keys.shape[1]
    rep = nq // nkv
    if rep > 1:
        keys = keys.repeat_interleave(rep, dim=1)
        values = values.repeat_interleave(rep, dim=1)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask {mask!r}")
        S = keys.shape[2]
        q_idx = torch.arange(S - L, S, device=queries.device)[:, None]
        mask = q_idx >= torch.arange(S, device=queries.device)[None]
    return torch.nn.functional.scaled_dot_product_attention(
        queries, keys, values, attn_mask=mask, scale=scale)


def create_causal_mask(N: int, offset: int = 0, window_size=None):
    q_idx = torch.arange(offset, offset + N)[:, None]
    k_idx = torch.arange(offset + N)[None]
    mask = q_idx >= k_idx
    if window_size is not None:
        mask = mask & (q_idx < k_idx + window_size)
    return mask


class KVCache:
    """Plain fp16 KV cache with the host-framework cache protocol."""

    step = 256

    def __init__(self):
        self.keys = None
        self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        B, H, S, D = keys.shape
        if self.keys is None or self.offset + S > self.keys.shape[2]:
            cap = ((self.offset + S + self.step - 1) // self.step) * self.step
            nk = torch.empty(B, H, cap, D, dtype=keys.dtype, device=keys.device)
            nv = torch.empty(B, H, cap, values.shape[3], dtype=values.dtype, device=values.device)
            if self.keys is not None and self.offset:
                nk[:, :, : self.offset] = self.keys[:, :, : self.offset]
                nv[:, :, : self.offset] = self.values[:, :, : self.offset]
            self.keys, self.values = nk, nv
        self.keys[:, :, self.offset: self.offset + S] = keys
        self.values[:, :, self.offset: self.offset + S] = values
        self.offset += S
        return self.keys[:, :, : self.offset], self.values[:, :, : self.offset]

    def make_mask(self, N, return_array=False, window_size=None, **kwargs):
        if N == 1:
            return None
        if return_array or (window_size and N > window_size):
            return create_causal_mask(N, offset=self.offset - N, window_size=window_size)
        return "causal"

    @property
    def state(self):
        if self.keys is None:
            return []
        return [self.keys[:, :, : self.offset], self.values[:, :, : self.offset]]

    @state.setter
    def state(self, v):
        self.keys, self.values = v
        self.offset = self.keys.shape[2]

    @property
    def meta_state(self):
        return ""

    @meta_state.setter
    def meta_state(self, v):
        pass

    def is_trimmable(self):
        return True

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        k, v = self.state
        return k.numel() * k.element_size() + v.numel() * v.element_size()


def make_prompt_cache(model):
    """One KVCache per attention layer of `model` (model.layers or model.n_layers)."""
    if hasattr(model, "make_cache"):
        return model.make_cache()
    n = len(model.layers) if hasattr(model, "layers") else int(model.n_layers)
    return [KVCache() for _ in range(n)]
