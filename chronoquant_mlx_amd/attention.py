"""ChronoQuant attention dispatch (reference attention.py:1-74).

Fused path: one query token per sequence over the compressed cache, run by
the gfx950 split-K decode kernel (cq_decode_attn).  The reference takes it
only for B == 1 (its Metal kernel has no batch axis); the gfx950 kernel has
one, so any batch size with q_len == 1 takes it here.

Prefill (q_len > 1, mask None or "causal", head_dim 128, fp16): the gfx950
chunked-prefill kernel (cq_prefill_attn), which computes the fallback's
semantics from the compressed cache without materialising K/V.

Fallback (array masks, other shapes): reconstruct fp16 K/V on the GPU
(cq_reconstruct) and run dense GQA attention with the reference's rounding
points: q' = fp16(q * fp16(scale)), fp16 scores, mask, softmax in fp32
rounded to the query dtype, fp16 weights @ V.
"""
from __future__ import annotations

import torch

from .kernels import (MAX_FUSED_HEAD_DIM, chronoquant_prefill_kernel, chronoquant_sdpa_cache_kernel,
                      prefill_supported)

# q_len > 1 with mask None / "causal" runs the gfx950 chunked-prefill kernel
# (same semantics as the reconstruct fallback below); False forces the
# fallback, which the tests use as a second implementation.
PREFILL_KERNEL = True


def _apply_mask(scores: torch.Tensor, mask):
    """attention.py:8-20."""
    if mask is None:
        return scores
    if isinstance(mask, str):
        q_len, k_len = scores.shape[-2:]
        q_idx = torch.arange(k_len - q_len, k_len, device=scores.device)
        k_idx = torch.arange(k_len, device=scores.device)
        mask = q_idx[:, None] >= k_idx[None]
    mask = mask.to(scores.device)
    if mask.dtype == torch.bool:
        return torch.where(mask, scores, torch.finfo(scores.dtype).min)
    return scores + mask.to(scores.dtype)


def chronoquant_sdpa(queries: torch.Tensor, keys, values, cache, scale: float, mask=None):
    """Attention over a ChronoQuantCache: the fused decode kernel for one
    query token, the chunked-prefill kernel, or GPU reconstruction + dense
    attention for everything else.

    queries: [B, n_q_heads, q_len, D]; keys/values are the placeholders
    update_and_fetch returned (attention reads the cache).
    """
    batch, n_q_heads, q_len, head_dim = queries.shape
    # bound to device positions (a graph-captured decode loop): the host
    # offset trails the device one, so only the fused decode reads the cache
    bound = getattr(cache, "_dev_pos", None) is not None
    use_fused = (
        cache.use_fused
        and q_len == 1
        and (cache.offset > 0 or bound)
        and head_dim <= MAX_FUSED_HEAD_DIM
        and (mask is None or (isinstance(mask, str) and mask == "causal"))
    )
    if bound and not use_fused:
        raise ValueError("a cache bound to device positions serves only the fused decode "
                         "(one query token, mask None, use_fused)")
    if use_fused:
        q = queries.reshape(batch, n_q_heads, head_dim)
        out = chronoquant_sdpa_cache_kernel(q, cache, scale, seq_lens=cache._dev_len)
        return out.reshape(batch, n_q_heads, q_len, head_dim)

    if PREFILL_KERNEL and prefill_supported(queries, cache, mask):
        return chronoquant_prefill_kernel(queries, cache, scale, causal=mask is not None)

    full_k, full_v = cache.reconstruct_history()
    n_kv_heads = full_k.shape[1]
    n_repeats = n_q_heads // n_kv_heads
    # weak-scalar semantics: scale is rounded to the query dtype first
    q_scaled = queries * torch.tensor(scale, dtype=queries.dtype, device=queries.device)
    q_grouped = q_scaled.reshape(batch, n_kv_heads, n_repeats, q_len, head_dim)
    dt = torch.promote_types(queries.dtype, full_k.dtype)
    k_t = full_k.to(dt).transpose(-1, -2).contiguous()[:, :, None]
    v_g = full_v.to(dt)[:, :, None]
    scores = torch.matmul(q_grouped.to(dt), k_t)
    scores = _apply_mask(scores, mask)
    weights = torch.softmax(scores.float(), dim=-1).to(dt)
    output = torch.matmul(weights, v_g)
    return output.reshape(batch, n_q_heads, q_len, head_dim).to(queries.dtype)
