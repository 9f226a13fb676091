"""INT4 packing helpers and the fused decode-attention operator.

Mirrors the reference module kernels.py (gauravsaini/chronoquant_mlx):
constants (kernels.py:5-7), pack_int4_codes (:34-54), unpack_int4_codes
(:57-61) and chronoquant_sdpa_kernel (:248-279), all backed by the gfx950
kernels of libchronoquant.so.
"""
from __future__ import annotations

import ctypes

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


def chronoquant_sdpa_cache_kernel(q: torch.Tensor, cache, scale: float = 1.0,
                                  out_dtype: torch.dtype | None = None,
                                  seq_lens: torch.Tensor | None = None,
                                  generic: bool = False) -> torch.Tensor:
    """Fused dequant + GQA decode attention over a ChronoQuantCache object,
    for B >= 1 (the form chronoquant_sdpa calls).

    q: [B, nq, D] (fp16 / bf16 / fp32) UNSCALED: the kernel forms q' =
    round(q * round(scale)) in q's dtype as attention.py:46 does.  seq_lens
    (int32 [B] on the device): per-sequence lengths, else cache.offset for
    every sequence.  Returns [B, nq, D] of out_dtype (default q.dtype).
    generic=True runs the portable kernel (a second GPU implementation).
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


def _rows_operand(t: torch.Tensor, name: str, row: int, dtype: torch.dtype):
    """A [H, n, row] (row > 1) or [H, n] (row == 1) kernel operand as (tensor,
    rows reserved per head): a view whose rows are contiguous and whose heads
    sit a whole number of rows apart is used in place (the cache's
    kernel_* slices are such views of its storage); anything else is copied
    contiguous."""
    if t.dtype != dtype:
        if dtype == torch.uint32 and t.dtype == torch.int32:
            t = t.view(torch.uint32)
        else:
            raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    want = 3 if row > 1 else 2
    if t.dim() != want or (row > 1 and t.shape[2] != row):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected [H, n{', ' + str(row) if row > 1 else ''}]")
    inner_ok = t.stride(-1) == 1 and (row == 1 or t.stride(1) == row)
    H, n = t.shape[0], t.shape[1]
    if inner_ok and H == 1:
        return t, max(n, 1)
    if inner_ok and t.stride(0) % row == 0 and t.stride(0) // row >= n:
        return t, t.stride(0) // row
    t = t.contiguous()
    return t, max(n, 1)


def chronoquant_sdpa_kernel(q: torch.Tensor, keyframes_k: torch.Tensor, packed_k: torch.Tensor,
                            scales_k: torch.Tensor, keyframes_v: torch.Tensor,
                            packed_v: torch.Tensor, scales_v: torch.Tensor, seq_len: int,
                            stride_k: int, stride_v: int) -> torch.Tensor:
    """Fused ChronoQuant SDPA for one sequence and one query token, with the
    reference operator's signature and contract (kernels.py:248-279).

    q: [n_q_heads, D], already scaled (attention.py:46 passes
    fp32(fp16(queries * scale))).  keyframes_*: fp16 [H, nkf, D]; packed_*:
    uint32 [H, npf, ceil(D/8)] INT4 words; scales_*: fp16 [H, npf] (the
    cache's kernel_*() slices, or the [H, 1, 1] / [H, 1] zero placeholders
    when a component has no P-frames).  Returns fp32 [n_q_heads, D].

    Semantics of the reference kernel: K/V dequantised in fp32 as a + c * s,
    fp32 softmax, q head j reads kv head j // (n_q_heads / H).  When q's
    values are fp16-representable (always, for the reference's caller) the
    MFMA decode runs on q as fp16; otherwise the portable kernel on fp32 q.
    """
    _lib.require_gpu(q)
    if q.dim() != 2:
        raise ValueError(f"q must be [n_q_heads, head_dim], got {tuple(q.shape)}")
    nq, D = q.shape
    H = keyframes_k.shape[0]
    seq_len, stride_k, stride_v = int(seq_len), int(stride_k), int(stride_v)
    if seq_len < 1 or stride_k < 1 or stride_v < 1:
        raise ValueError("seq_len and the strides must be >= 1")
    W = (D + 7) // 8
    dev = q.device
    comps = []
    for c, kf, pk, sc, s in (("k", keyframes_k, packed_k, scales_k, stride_k),
                             ("v", keyframes_v, packed_v, scales_v, stride_v)):
        nkf = (seq_len - 1) // s + 1
        npf = seq_len - nkf
        kf, cap_kf = _rows_operand(kf, f"keyframes_{c}", D, torch.float16)
        if kf.shape[0] != H or kf.shape[1] < nkf:
            raise ValueError(f"keyframes_{c} {tuple(kf.shape)} holds fewer than the {nkf} "
                             f"anchors of seq_len {seq_len}")
        if npf == 0:
            # the reference's placeholders (or anything): no P-frame is read
            pk = torch.zeros(H, 1, W, dtype=torch.uint32, device=dev)
            sc = torch.zeros(H, 1, dtype=torch.float16, device=dev)
        pk, cap_pk = _rows_operand(pk, f"packed_{c}", W, torch.uint32)
        sc, cap_sc = _rows_operand(sc, f"scales_{c}", 1, torch.float16)
        if pk.shape[0] != H or sc.shape[0] != H or pk.shape[1] < npf or sc.shape[1] < npf:
            raise ValueError(f"packed_{c} / scales_{c} hold fewer than the {npf} P-frames of "
                             f"seq_len {seq_len}")
        if cap_pk != cap_sc:  # one row capacity per component in the descriptor
            pk, sc = pk.contiguous(), sc.contiguous()
            cap_pk = cap_sc = max(pk.shape[1], 1)
        for t in (kf, pk, sc):
            if t.device != dev:
                raise ValueError("every operand must be on q's device")
        comps.append((kf, pk, sc, cap_kf, cap_pk, s))
    d = _lib.CqCacheDesc()
    d.batch, d.n_kv_heads, d.head_dim = 1, H, D
    for comp, (kf, pk, sc, cap_kf, cap_pf, s) in zip((d.k, d.v), comps):
        comp.keyframes, comp.packed, comp.scales = kf.data_ptr(), pk.data_ptr(), sc.data_ptr()
        comp.cap_keyframes, comp.cap_pframes = cap_kf, cap_pf
        comp.stride, comp.delta_bits, comp.dead_zone = s, 4, 0.0
    if q.dtype == torch.float32 and torch.equal(q.half().float(), q):
        qk = q.half().contiguous()
    else:
        qk = q.contiguous()
    out = torch.empty(nq, D, dtype=torch.float32, device=dev)
    from .cache import _shared_workspace
    need = _lib.load().cq_decode_workspace_size(1, H, nq, D, seq_len)
    ws = _shared_workspace(dev, need)
    _lib.call("cq_decode_attn", ctypes.byref(d), qk.data_ptr(), _lib.dtype_code(qk.dtype), nq, 1.0,
              None, seq_len, seq_len, out.data_ptr(), _lib.CQ_F32, ws.data_ptr(), ws.numel(),
              _lib.stream_of(q))
    return out


def decode_status(workspace: torch.Tensor | None = None) -> int:
    """cq_decode_status: 0, or CQ_ERR_TIMEOUT when a split wait of an earlier
    decode on this workspace (None: the current device's no-alloc scratch)
    ran out of poll rounds; the workspace's split state is then cleared.
    Synchronises the current stream."""
    stream = torch.cuda.current_stream().cuda_stream
    return _lib.load().cq_decode_status(_lib.ptr(workspace), stream)


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
    dense = any(cache._packing(c) != _lib.CQ_PACK_INT4 for c in ("k", "v"))
    return (L > 1 and D == 128 and not dense and queries.dtype in (torch.float16, torch.bfloat16)
            and (mask is None or (isinstance(mask, str) and mask == "causal"))
            and cache.offset >= L and nq % cache._shape[1] == 0
            and 256 % (nq // cache._shape[1]) == 0)
