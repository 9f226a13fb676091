"""INT4 packing helpers and the fused decode-attention operator.

Mirrors the reference module kernels.py (gauravsaini/chronoquant_mlx):
constants (kernels.py:5-7), pack_int4_codes (:34-54), unpack_int4_codes
(:57-61) and chronoquant_sdpa_kernel (:248-279), all backed by the gfx950
kernels of libchronoquant.so.
"""
from __future__ import annotations

import torch

from . import _lib

MAX_FUSED_HEAD_DIM = 256  # kernels.py:5
# The reference's Metal launch shape (kernels.py:6-7): 31 simdgroups of 32
# lanes per q head.  The gfx950 kernels launch split-K workgroups of 4 wave64
# instead; the names are kept for API compatibility.
FUSED_SIMDGROUPS = 31
FUSED_THREADGROUP_SIZE = FUSED_SIMDGROUPS * 32


def pack_int4_codes(codes: torch.Tensor) -> torch.Tensor:
    """Pack signed INT4 codes [-8, 7] into uint32 words (kernels.py:34-54).

    codes: int8 [..., D] on the GPU -> uint32 [..., ceil(D/8)]; nibble i of a
    word holds clip(code + 8, 0, 15) of dim 8w+i; D is padded with nibble 0.
    """
    _lib.require_gpu(codes)
    if codes.dtype != torch.int8:
        codes = codes.to(torch.int8)
    codes = codes.contiguous()
    D = codes.shape[-1]
    W = (D + 7) // 8
    out = torch.empty(*codes.shape[:-1], W, dtype=torch.uint32, device=codes.device)
    rows = codes.numel() // D if D else 0
    _lib.call("cq_pack_int4", codes.data_ptr(), rows, D, out.data_ptr(), _lib.stream_of(codes))
    return out


def unpack_int4_codes(packed: torch.Tensor, head_dim: int) -> torch.Tensor:
    """Unpack uint32 words back to signed INT4 codes [-8, 7] (kernels.py:57-61)."""
    _lib.require_gpu(packed)
    if packed.dtype != torch.uint32:
        packed = packed.view(torch.uint32) if packed.dtype == torch.int32 else packed.to(torch.uint32)
    packed = packed.contiguous()
    W = packed.shape[-1]
    if (head_dim + 7) // 8 > W:
        raise ValueError(f"head_dim {head_dim} needs {(head_dim + 7) // 8} words, got {W}")
    out = torch.empty(*packed.shape[:-1], head_dim, dtype=torch.int8, device=packed.device)
    rows = packed.numel() // W if W else 0
    if W * 8 != ((head_dim + 7) // 8) * 8:
        # rows carry extra words: unpack the leading ceil(head_dim/8) of each
        packed = packed[..., : (head_dim + 7) // 8].contiguous()
    _lib.call("cq_unpack_int4", packed.data_ptr(), rows, head_dim, out.data_ptr(),
              _lib.stream_of(packed))
    return out


def chronoquant_sdpa_kernel(q: torch.Tensor, cache, scale: float = 1.0,
                            out_dtype: torch.dtype | None = None,
                            seq_lens: torch.Tensor | None = None,
                            generic: bool = False) -> torch.Tensor:
    """Fused dequant + GQA decode attention over a ChronoQuantCache.

    Counterpart of chronoquant_sdpa_kernel (kernels.py:248-279) taking the
    cache object instead of its squeezed slices, and B >= 1.  q: [B, nq, D]
    (fp16 / bf16 / fp32) UNSCALED: the kernel forms q' = round(q * round(scale))
    in q's dtype as attention.py:46 does.  Returns [B, nq, D] of out_dtype
    (default q.dtype).
    """
    _lib.require_gpu(q)
    q = q.contiguous()
    B, nq, D = q.shape
    out = torch.empty(B, nq, D, dtype=out_dtype or q.dtype, device=q.device)
    desc = cache._descriptor()
    ws = cache._decode_workspace(nq)
    if seq_lens is not None:
        lens = seq_lens
        if lens.device != q.device or lens.dtype != torch.int32 or not lens.is_contiguous():
            lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
        max_len = int(cache._max_len)
        lens_ptr = lens.data_ptr()
    else:
        lens_ptr, max_len = None, cache.offset
    fn = "cq_decode_attn_generic" if generic else "cq_decode_attn"
    _lib.call(fn, desc, q.data_ptr(), _lib.dtype_code(q.dtype), nq, float(scale), lens_ptr,
              cache.offset, max_len, out.data_ptr(), _lib.dtype_code(out.dtype),
              ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    return out


def chronoquant_prefill_kernel(q: torch.Tensor, cache, scale: float = 1.0,
                               causal: bool = True) -> torch.Tensor:
    """Chunked-prefill attention over a ChronoQuantCache (cq_prefill_attn).

    q: [B, nq, L, 128] fp16 or bf16 UNSCALED; the L queries are the cache's
    last L tokens (already appended).  Causal (query i sees keys <= offset -
    L + i) or full attention.  Same result semantics as the reconstruct
    fallback of chronoquant_sdpa (attention.py:61-74).  Returns
    [B, nq, L, 128] of q's dtype.
    """
    _lib.require_gpu(q)
    q = q.contiguous()
    B, nq, L, D = q.shape
    out = torch.empty_like(q)
    ws = cache._prefill_workspace(nq, L)
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    _lib.call("cq_prefill_attn", cache._descriptor(), q.data_ptr(), _lib.dtype_code(q.dtype), nq,
              L, float(scale), int(bool(causal)), cache.offset, out.data_ptr(), ws_ptr, ws_bytes,
              _lib.stream_of(q))
    return out


def prefill_supported(queries: torch.Tensor, cache, mask) -> bool:
    """Whether cq_prefill_attn serves this chronoquant_sdpa call."""
    B, nq, L, D = queries.shape
    return (L > 1 and D == 128 and queries.dtype in (torch.float16, torch.bfloat16)
            and (mask is None or (isinstance(mask, str) and mask == "causal"))
            and cache.offset >= L and nq % cache._shape[1] == 0
            and 256 % (nq // cache._shape[1]) == 0)
