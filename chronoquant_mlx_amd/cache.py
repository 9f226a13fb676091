"""ChronoQuant KV cache on the GPU (PyTorch-ROCm storage, HIP kernels).

Mirrors ChronoQuantCache (reference cache.py:18-287): token t is an I-frame
(fp16 anchor) iff t % stride == 0, otherwise a P-frame holding its INT4
residual against anchor t // stride; K and V use independent strides, bit
widths and dead zones.  Differences in mechanism (not in results):

* storage is allocated with spare capacity and appended in place by one
  fused HIP launch per update (codec + pack + I-frame store for K and V),
  instead of a per-token Python loop and a full-history concatenate;
* update_and_fetch does not synchronise the host (the reference calls
  mx.eval there); the work is ordered on the current HIP stream.

The active prefix of every storage tensor equals the reference's tensor, so
`state`, `nbytes` and the kernel_* accessors return the reference's values.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .codec import ChronoQuantCodec

_GROW_QUANTUM = 256  # tokens


def make_causal_mask(offset: int, num_queries: int, return_array: bool = False,
                     window_size=None):
    """cache.py:7-15: None for one query, "causal" otherwise; an explicit
    boolean mask [num_queries, offset] when asked for (or windowed)."""
    if num_queries == 1:
        return None
    if return_array or (window_size and num_queries > window_size):
        q_idx = torch.arange(offset - num_queries, offset)[:, None]
        k_idx = torch.arange(offset)[None, :]
        mask = q_idx >= k_idx
        if window_size is not None:
            mask = mask & (q_idx < k_idx + window_size)
        return mask
    return "causal"


def _num_keyframes(num_tokens: int, stride: int) -> int:
    return 0 if num_tokens <= 0 else (num_tokens - 1) // stride + 1


def _num_pframes(num_tokens: int, stride: int) -> int:
    return num_tokens - _num_keyframes(num_tokens, stride)


_WORKSPACES: dict = {}
# Workspaces replaced by larger ones.  A captured HIP graph keeps the address
# it was captured with, so a replaced workspace is never freed.
_RETIRED: list = []
# Workspaces allocated under stream capture, one per capture (key: device,
# stream, capture id); kept for the life of the process with their graphs.
_CAPTURE_WORKSPACES: dict = {}


def _shared_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised split-K workspace of the decode and prefill kernels,
    one per (device, stream): the caches that run on one stream share it.

    The kernels return its counters to zero, so it is reused without
    clearing.  Calls on one stream are ordered, so they never overlap on
    it; calls on another stream use another workspace.

    Under stream capture a graph gets a workspace of its own, allocated from
    the graph's memory pool at its first use in the capture (the zero fill is
    a kernel captured with it, so every replay starts from zeroed counters)
    and shared only by the calls of that capture.  A capture never reuses the
    stream's eager workspace (a graph may be replayed on another stream,
    concurrently with eager calls) and eager calls never see a capture's.
    """
    stream = torch.cuda.current_stream(device)
    handle = stream.cuda_stream
    cid = _lib.stream_capture_id(handle) if torch.cuda.is_current_stream_capturing() else None
    table = _WORKSPACES if cid is None else _CAPTURE_WORKSPACES
    key = (device.index, handle) if cid is None else (device.index, handle, cid)
    ws = table.get(key)
    if ws is None or ws.numel() < nbytes:
        old = 0 if ws is None else ws.numel()
        new = torch.zeros(max(nbytes, 1 << 20, 2 * old), dtype=torch.uint8, device=device)
        if ws is not None:
            _RETIRED.append(ws)
        table[key] = ws = new
    return ws


def dense_rows_of_int4(words: torch.Tensor, head_dim: int, bits: int) -> torch.Tensor:
    """INT4-lane rows [..., ceil(D/8)] -> dense rows [..., ceil(D * bits / 32)]
    (the layout CQ_PACK_DENSE components hold in HBM: the little-endian
    stream of persist.dense_pack, zero-padded to whole words)."""
    from .persist import dense_pack
    stream = dense_pack(words.contiguous(), head_dim, bits)
    rw = (head_dim * bits + 31) // 32
    pad = 4 * rw - stream.shape[-1]
    if pad:
        stream = torch.nn.functional.pad(stream, (0, pad))
    return stream.contiguous().view(torch.uint32)


def int4_of_dense_rows(rows: torch.Tensor, head_dim: int, bits: int) -> torch.Tensor:
    """Inverse of dense_rows_of_int4."""
    from .persist import dense_unpack
    nbytes = (head_dim * bits + 7) // 8
    return dense_unpack(rows.contiguous().view(torch.uint8)[..., :nbytes], head_dim, bits)


class ChronoQuantCache:
    """KV cache of fp16 anchors (every stride-th token) and INT4-coded
    residual rows for the tokens between them, read by the fused decode."""

    def __init__(
        self,
        stride_k: int = 32,
        stride_v: int = 8,
        delta_bits_k: int = 4,
        delta_bits_v: int = 4,
        dead_zone_k: float = 0.0,
        dead_zone_v: float = 0.05,
        use_fused: bool = True,
        per_layer_v_bits: list = None,
        layer_idx: int = 0,
        capacity: int = 0,
        dense_residuals: bool = False,
    ):
        if stride_k < 1 or stride_v < 1:
            raise ValueError("strides must be >= 1")
        self.stride_k = stride_k
        self.stride_v = stride_v
        self.delta_bits_k = delta_bits_k
        self.delta_bits_v = delta_bits_v
        self.dead_zone_k = dead_zone_k
        self.dead_zone_v = dead_zone_v
        self.use_fused = use_fused
        # opt-in: 2- and 3-bit components keep their codes at their own width
        # in HBM (this library's format; the reference's rows are INT4 lanes)
        self.dense_residuals = bool(dense_residuals)
        self.per_layer_v_bits = per_layer_v_bits or []
        self.layer_idx = layer_idx
        self.codec_k = ChronoQuantCodec(stride=stride_k, delta_bits=delta_bits_k,
                                        dead_zone_ratio=dead_zone_k)
        self._codec_v = None
        self.offset = 0
        self.head_dim = None
        self._initial_capacity = int(capacity)
        self._cap = 0
        self._shape = None  # (B, H, D)
        self._device = None
        self._kf = {"k": None, "v": None}
        self._pk = {"k": None, "v": None}
        self._sc = {"k": None, "v": None}
        self._max_len = 0
        self._dev_pos = None  # device positions (bind_device_position)
        self._dev_len = None
        self._len_owner = True  # this cache computes _dev_len = pos + S

    # ------------------------------------------------------------------
    # counting (cache.py:53-61)
    # ------------------------------------------------------------------
    @staticmethod
    def _num_keyframes(num_tokens: int, stride: int) -> int:
        return _num_keyframes(num_tokens, stride)

    @classmethod
    def _num_pframes(cls, num_tokens: int, stride: int) -> int:
        return _num_pframes(num_tokens, stride)

    def _stride(self, component: str) -> int:
        return self.stride_k if component == "k" else self.stride_v

    def _bits(self, component: str) -> int:
        return self.delta_bits_k if component == "k" else self._get_codec_for_v().delta_bits

    def _packing(self, component: str) -> int:
        """CQ_PACK_DENSE for a 2- or 3-bit component of a dense_residuals
        cache, else CQ_PACK_INT4 (the reference's layout)."""
        dense = self.dense_residuals and self._bits(component) < 4
        return _lib.CQ_PACK_DENSE if dense else _lib.CQ_PACK_INT4

    def _row_words(self, component: str) -> int:
        """uint32 words of one packed row: ceil(D/8) in INT4 lanes, ceil(D *
        bits / 32) for dense rows."""
        D = self._shape[2]
        fb = self._bits(component) if self._packing(component) == _lib.CQ_PACK_DENSE else 4
        return (D * fb + 31) // 32

    # ------------------------------------------------------------------
    # active views (cache.py:63-85)
    # ------------------------------------------------------------------
    def _active_keyframes(self, component: str):
        t = self._kf[component]
        if t is None:
            return None
        return t[:, :, : _num_keyframes(self.offset, self._stride(component)), :]

    def _active_packed(self, component: str):
        t = self._pk[component]
        if t is None:
            return None
        return t[:, :, : _num_pframes(self.offset, self._stride(component)), :]

    def _active_scales(self, component: str):
        t = self._sc[component]
        if t is None:
            return None
        return t[:, :, : _num_pframes(self.offset, self._stride(component))]

    # reference attribute names (cache.py:46-51) as active views
    keyframes_k = property(lambda self: self._active_keyframes("k"))
    keyframes_v = property(lambda self: self._active_keyframes("v"))
    packed_codes_k = property(lambda self: self._active_packed("k"))
    packed_codes_v = property(lambda self: self._active_packed("v"))
    pframe_scales_k = property(lambda self: self._active_scales("k"))
    pframe_scales_v = property(lambda self: self._active_scales("v"))

    # ------------------------------------------------------------------
    # storage
    # ------------------------------------------------------------------
    def _allocate(self, cap: int):
        B, H, D = self._shape
        dev = self._device
        for c in ("k", "v"):
            W = self._row_words(c)
            s = self._stride(c)
            nkf = max(1, _num_keyframes(cap, s))
            npf = max(1, _num_pframes(cap, s))
            kf = torch.empty(B, H, nkf, D, dtype=torch.float16, device=dev)
            pk = torch.empty(B, H, npf, W, dtype=torch.uint32, device=dev)
            sc = torch.empty(B, H, npf, dtype=torch.float16, device=dev)
            old = (self._kf[c], self._pk[c], self._sc[c])
            if old[0] is not None and self.offset > 0:
                n_kf = _num_keyframes(self.offset, s)
                n_pf = _num_pframes(self.offset, s)
                kf[:, :, :n_kf].copy_(old[0][:, :, :n_kf])
                if n_pf:
                    pk[:, :, :n_pf].copy_(old[1][:, :, :n_pf])
                    sc[:, :, :n_pf].copy_(old[2][:, :, :n_pf])
            self._kf[c], self._pk[c], self._sc[c] = kf, pk, sc
        self._cap = cap

    def _ensure_capacity(self, needed: int):
        if needed <= self._cap:
            return
        cap = max(needed, 2 * self._cap, self._initial_capacity, _GROW_QUANTUM)
        cap = (cap + _GROW_QUANTUM - 1) // _GROW_QUANTUM * _GROW_QUANTUM
        self._allocate(cap)

    def reserve(self, num_tokens: int):
        """Pre-allocate room for num_tokens tokens (no reference counterpart)."""
        if self._shape is None:
            self._initial_capacity = max(self._initial_capacity, int(num_tokens))
        else:
            self._ensure_capacity(int(num_tokens))

    def _get_codec_for_v(self):
        """cache.py:192-196 (lazy V codec, per-layer bits)."""
        if self._codec_v is None:
            if self.per_layer_v_bits:
                v_bits = self.per_layer_v_bits[min(self.layer_idx, len(self.per_layer_v_bits) - 1)]
            else:
                v_bits = self.delta_bits_v
            self._codec_v = ChronoQuantCodec(stride=self.stride_v, delta_bits=v_bits,
                                             dead_zone_ratio=self.dead_zone_v)
        return self._codec_v

    def _descriptor(self) -> "_lib.CqCacheDesc":
        B, H, D = self._shape
        d = _lib.CqCacheDesc()
        d.batch, d.n_kv_heads, d.head_dim = B, H, D
        codecs = {"k": self.codec_k, "v": self._get_codec_for_v()}
        for c in ("k", "v"):
            comp = getattr(d, c)
            comp.keyframes = self._kf[c].data_ptr()
            comp.packed = self._pk[c].data_ptr()
            comp.scales = self._sc[c].data_ptr()
            comp.cap_keyframes = self._kf[c].shape[2]
            comp.cap_pframes = self._pk[c].shape[2]
            comp.stride = self._stride(c)
            comp.delta_bits = codecs[c].delta_bits
            comp.dead_zone = float(codecs[c].dead_zone_ratio)
            comp.packing = self._packing(c)
        return ctypes.byref(d)

    def _decode_workspace(self, n_q_heads: int) -> torch.Tensor:
        B, H, D = self._shape
        need = _lib.load().cq_decode_workspace_size(B, H, n_q_heads, D, max(self._cap, 1))
        return _shared_workspace(self._device, need)

    def _prefill_workspace(self, n_q_heads: int, n_q: int) -> torch.Tensor | None:
        """Split-K workspace of cq_prefill_attn (the shared decode workspace,
        grown when needed); None when the plan does not split."""
        B, H, D = self._shape
        need = _lib.load().cq_prefill_workspace_size(B, H, n_q_heads, n_q, max(self.offset, 1))
        return _shared_workspace(self._device, need) if need else None

    # ------------------------------------------------------------------
    # append (cache.py:87-129, 198-215)
    # ------------------------------------------------------------------
    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Compress new KV states and return lightweight placeholders."""
        B, H, S, head_dim = keys.shape
        if self.head_dim is None:
            self.head_dim = head_dim
        elif head_dim != self.head_dim:
            raise ValueError(f"ChronoQuantCache head_dim changed: {self.head_dim} -> {head_dim}")
        if values.shape != keys.shape:
            raise ValueError(f"keys {tuple(keys.shape)} and values {tuple(values.shape)} differ")
        if values.dtype != keys.dtype:
            raise TypeError("keys and values must share a dtype")
        _lib.require_gpu(keys)
        if self._shape is None:
            self._shape = (B, H, head_dim)
            self._device = keys.device
        elif self._shape[:2] != (B, H):
            raise ValueError(f"ChronoQuantCache batch/heads changed: {self._shape[:2]} -> {(B, H)}")
        if S == 0:
            return keys, values
        if keys.stride(-1) != 1:
            keys = keys.contiguous()
        if values.stride(-1) != 1:
            values = values.contiguous()
        ks = (ctypes.c_int64 * 3)(keys.stride(0), keys.stride(1), keys.stride(2))
        vs = (ctypes.c_int64 * 3)(values.stride(0), values.stride(1), values.stride(2))
        if self._dev_pos is not None:
            # device positions: append at pos[b], the fused decode reads
            # pos[b] + S tokens (chronoquant_sdpa serves a bound cache with
            # the fused decode only: its other paths read the host offset)
            _lib.call("cq_append", self._descriptor(), keys.data_ptr(), ks, values.data_ptr(), vs,
                      _lib.dtype_code(keys.dtype), S, self._dev_pos.data_ptr(), 0,
                      _lib.stream_of(keys))
            if self._len_owner:
                torch.add(self._dev_pos, S, out=self._dev_len)
            return keys, values
        self._ensure_capacity(self.offset + S)
        _lib.call("cq_append", self._descriptor(), keys.data_ptr(), ks, values.data_ptr(), vs,
                  _lib.dtype_code(keys.dtype), S, None, self.offset, _lib.stream_of(keys))
        self.offset += S
        self._max_len = self.offset
        return keys, values

    def fused_decode_append(self, qkv: torch.Tensor, n_q_heads: int,
                            q_weight: torch.Tensor | None, k_weight: torch.Tensor | None,
                            cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                            eps: float) -> torch.Tensor | None:
        """One new token per sequence straight from a fused QKV projection
        qkv [B, 1, (n_q_heads + 2 H) * 128]: RMSNorm and rotary embedding of
        the query and key heads, and the append of the key and value heads,
        in one launch (cq_qkv_rope_append).  The same bits as
        fused.qkv_norm_rope followed by update_and_fetch (cache.py:198-215 in
        the reference; no counterpart for the fusion).  Returns q [B,
        n_q_heads, 1, 128], or None when the cache cannot take the token this
        way (not shaped by an earlier append, another head_dim, batch or head
        count): the caller then runs the two steps."""
        if self._shape is None:
            return None
        B, H, D = self._shape
        if D != 128 or qkv.shape != (B, 1, (n_q_heads + 2 * H) * D) or qkv.device != self._device:
            return None
        for t in (cos, sin):
            if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != D // 2 or t.device != qkv.device:
                raise ValueError("fused_decode_append: cos/sin must be fp32 [max_pos, 64] on qkv's device")
        for w in (q_weight, k_weight):
            if w is not None and (w.shape != (D,) or w.dtype != qkv.dtype or w.device != qkv.device):
                raise ValueError("fused_decode_append: norm weights must be [128] of qkv's dtype")
        positions = positions.to(device=qkv.device, dtype=torch.int64)
        if positions.numel() == 1:
            bstride = 0
        elif positions.shape in ((B,), (B, 1)):
            bstride = 1
        else:
            raise ValueError("fused_decode_append: positions must be [1], [B] or [B, 1]")
        qkv, cos, sin, positions = qkv.contiguous(), cos.contiguous(), sin.contiguous(), positions.contiguous()
        q = torch.empty(B, n_q_heads, 1, D, dtype=qkv.dtype, device=qkv.device)
        if self._dev_pos is not None:
            offsets, offset = self._dev_pos.data_ptr(), 0
            lengths = self._dev_len.data_ptr() if self._len_owner else None
        else:
            self._ensure_capacity(self.offset + 1)
            offsets, offset, lengths = None, self.offset, None
        _lib.call("cq_qkv_rope_append", self._descriptor(), qkv.data_ptr(), _lib.ptr(q_weight),
                  _lib.ptr(k_weight), q.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                  positions.data_ptr(), bstride, n_q_heads, float(eps),
                  _lib.dtype_code(qkv.dtype), offsets, offset, lengths, _lib.stream_of(qkv))
        if self._dev_pos is None:
            self.offset += 1
            self._max_len = self.offset
        return q

    # ------------------------------------------------------------------
    # device positions (graph-captured serving loops; no reference counterpart)
    # ------------------------------------------------------------------
    def bind_device_position(self, pos: torch.Tensor | None, max_len: int = 0,
                             lengths: torch.Tensor | None = None,
                             update_lengths: bool = True):
        """Take positions from device memory instead of the host offset.

        With `pos` (int32 [B], on the cache's device) bound, update_and_fetch
        appends sequence b's new tokens at pos[b].. and the fused decode reads
        pos[b] + S tokens.  No host value changes between steps, so a captured
        HIP graph of a decode step replays at successive positions.  The
        caller advances pos on the device and the host-side offset with
        advance() after each step.  Room for max_len tokens is reserved now
        (no reallocation may happen under capture).  pos=None returns to host
        offsets.

        Caches stepped together (the layers of one model) can share the
        per-sequence length vector pos + S: pass the same `lengths` tensor
        to each and let one of them (update_lengths=True, appended first in
        every step) compute it.
        """
        if pos is None:
            self._dev_pos = self._dev_len = None
            self._len_owner = True
            self._max_len = self.offset
            return
        if pos.dtype != torch.int32 or pos.dim() != 1:
            raise TypeError("pos must be an int32 vector [B]")
        if lengths is not None and (lengths.shape != pos.shape or lengths.dtype != pos.dtype
                                    or lengths.device != pos.device):
            raise TypeError("lengths must match pos (int32 [B], same device)")
        self.reserve(max_len)
        self._dev_pos = pos
        self._dev_len = torch.empty_like(pos) if lengths is None else lengths
        self._len_owner = lengths is None or bool(update_lengths)
        self._max_len = int(max_len)

    def advance(self, n: int):
        """Host-side offset after n tokens were appended at device positions."""
        self.offset += int(n)

    # ------------------------------------------------------------------
    # reconstruction (cache.py:131-160)
    # ------------------------------------------------------------------
    def _reconstruct_component(self, component: str):
        if self.offset == 0:
            return None
        B, H, D = self._shape
        out = torch.empty(B, H, self.offset, D, dtype=torch.float16, device=self._device)
        cid = _lib.CQ_KEYS if component == "k" else _lib.CQ_VALUES
        _lib.call("cq_reconstruct", self._descriptor(), cid, self.offset, out.data_ptr(),
                  _lib.stream_of(out))
        return out

    def reconstruct_history(self):
        """fp16 K and V of every cached token, [B, H, offset, D] each, for the
        attention paths that do not read the compressed rows directly."""
        return self._reconstruct_component("k"), self._reconstruct_component("v")

    # ------------------------------------------------------------------
    # kernel operand accessors (cache.py:162-190), B == 1
    # ------------------------------------------------------------------
    def kernel_keyframes_k(self):
        return self._active_keyframes("k").squeeze(0)

    def kernel_keyframes_v(self):
        return self._active_keyframes("v").squeeze(0)

    def _kernel_packed(self, c):
        """(Dense rows for a dense_residuals component: the reference
        operator's INT4 reading does not apply to them.)"""
        p = self._active_packed(c)
        if p is not None and p.shape[2] > 0:
            return p.squeeze(0)
        return torch.zeros(self._shape[1], 1, 1, dtype=torch.uint32, device=self._device)

    def _kernel_scales(self, c):
        s = self._active_scales(c)
        if s is not None and s.shape[2] > 0:
            return s.squeeze(0)
        return torch.zeros(self._shape[1], 1, dtype=torch.float16, device=self._device)

    def kernel_packed_k(self):
        return self._kernel_packed("k")

    def kernel_packed_v(self):
        return self._kernel_packed("v")

    def kernel_scales_k(self):
        return self._kernel_scales("k")

    def kernel_scales_v(self):
        return self._kernel_scales("v")

    # ------------------------------------------------------------------
    # host-framework cache protocol (cache.py:217-287)
    # ------------------------------------------------------------------
    def make_mask(self, num_queries, return_array=False, window_size=None, **kwargs):
        return make_causal_mask(self.offset, num_queries, return_array, window_size)

    @property
    def state(self):
        """[keyframes_k, keyframes_v, packed_k, scales_k, packed_v, scales_v].

        The reference (cache.py:220-234) omits a component's packed/scales pair
        while it has no P-frames, which makes a 4-tensor list ambiguous
        (stride_k=1); this cache always emits all six (empty when unused).
        A dense_residuals component's packed tensor holds its dense rows.
        """
        if self.offset == 0 or self._kf["k"] is None:
            return []
        return [self._active_keyframes("k"), self._active_keyframes("v"),
                self._active_packed("k"), self._active_scales("k"),
                self._active_packed("v"), self._active_scales("v")]

    @state.setter
    def state(self, values):
        """Restore from a state list (cache.py:236-255).  Six tensors are read
        in the order above; shorter lists follow the reference's reading.
        Packed rows may be INT4 words (the reference's state) or, for a
        dense_residuals component, its dense rows; INT4 words given to a dense
        component are converted."""
        if not values:
            return
        kf_k, kf_v = values[0], values[1]
        pk_k = sc_k = pk_v = sc_v = None
        if len(values) >= 6:
            pk_k, sc_k, pk_v, sc_v = values[2], values[3], values[4], values[5]
        elif len(values) >= 4:
            # The reference emits a component's packed/scales pair only when
            # it has P-frames (cache.py:227-231) but reads a lone pair as the
            # keys' (cache.py:243-246).  With stride_k == 1 the keys never
            # have P-frames, so a lone pair can only be the values'.
            if self.stride_k == 1 and self.stride_v > 1:
                pk_v, sc_v = values[2], values[3]
            else:
                pk_k, sc_k = values[2], values[3]
        B, H, _, D = kf_k.shape
        self.head_dim = D
        self._shape = (B, H, D)
        self._device = kf_k.device
        _lib.require_gpu(kf_k)
        n_pk = 0 if pk_k is None else pk_k.shape[2]
        offset = kf_k.shape[2] + n_pk  # cache.py:254-255
        if (_num_keyframes(offset, self.stride_k) != kf_k.shape[2]
                or _num_keyframes(offset, self.stride_v) != kf_v.shape[2]):
            raise ValueError("state tensors do not match this cache's strides")
        self.offset = 0
        self._kf = {"k": None, "v": None}
        self._pk = {"k": None, "v": None}
        self._sc = {"k": None, "v": None}
        self._cap = 0
        self._ensure_capacity(max(offset, 1))
        for c, kf, pk, sc in (("k", kf_k, pk_k, sc_k), ("v", kf_v, pk_v, sc_v)):
            self._kf[c][:, :, : kf.shape[2]].copy_(kf.to(torch.float16))
            n_pf = _num_pframes(offset, self._stride(c))
            if n_pf:
                rw = self._row_words(c)
                if pk is None or pk.shape[2] != n_pf or pk.shape[3] not in (rw, (D + 7) // 8):
                    raise ValueError(f"state is missing the {c} P-frames")
                pk = pk.view(torch.uint32) if pk.dtype == torch.int32 else pk
                if pk.shape[3] != rw:  # INT4 words for a dense component
                    pk = dense_rows_of_int4(pk.to(self._device), D, self._bits(c))
                self._pk[c][:, :, :n_pf].copy_(pk)
                self._sc[c][:, :, :n_pf].copy_(sc.reshape(B, H, n_pf).to(torch.float16))
        self.offset = offset
        self._max_len = offset

    @property
    def meta_state(self):
        return ""

    @meta_state.setter
    def meta_state(self, value):
        pass

    def is_trimmable(self):
        return False

    def empty(self):
        return self.offset == 0

    def has_previous_state(self) -> bool:
        return self.offset > 0

    @property
    def nbytes(self) -> int:
        """Active bytes of the six storage tensors (cache.py:274-287)."""
        total = 0
        for c in ("k", "v"):
            for t in (self._active_keyframes(c), self._active_packed(c), self._active_scales(c)):
                if t is not None:
                    total += t.numel() * t.element_size()
        return total
