"""Second, independent CPU restatement of the ChronoQuant codec (numpy).

TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check the C oracle
(oracle/cq_oracle.c) bit for bit and to write the golden fixtures under
tests/golden/.  The product path never imports it.

numpy float16 arithmetic rounds each elementwise result to binary16 with
round-to-nearest-even, which is the arithmetic model of MLX fp16 arrays; bf16
is emulated by rounding a float32 result to bfloat16 after every operation.
Functions follow the reference (gauravsaini/chronoquant_mlx) line by line:

    quantize_delta      codec.py:23-65
    dequantize_delta    codec.py:67-73
    pack_int4_codes     kernels.py:34-54 (MSL kernels.py:9-22)
    unpack_int4_codes   kernels.py:57-61
    append / reconstruct cache.py:87-156 (one sequence, [H, S, D] tokens)
    sdpa_fallback       attention.py:8-20, 61-74
"""
from __future__ import annotations

import numpy as np

F16, BF16, F32 = "f16", "bf16", "f32"


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even), returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class _Arith:
    """Elementwise arithmetic of one array dtype: every result is rounded."""

    def __init__(self, dtype: str):
        self.dtype = dtype

    def r(self, x):
        x = np.asarray(x, dtype=np.float32)
        if self.dtype == F16:
            return x.astype(np.float16).astype(np.float32)
        if self.dtype == BF16:
            return bf16_bits_to_f32(f32_to_bf16_bits(x))
        return x

    def scalar(self, s: float) -> np.float32:
        # weak Python scalar: converted to the array dtype
        if self.dtype == F16:
            return np.float32(np.float16(s))
        if self.dtype == BF16:
            return self.r(np.float32(s))[()]
        return np.float32(s)


def quantize_delta(delta: np.ndarray, delta_bits: int, dead_zone: float,
                   dtype: str = F16):
    """codec.py:23-65.  delta: float32 array holding `dtype` values, [..., D].

    Returns (codes int8 [..., D], scales fp16 [..., 1]).
    """
    A = _Arith(dtype)
    half = (2 ** delta_bits) // 2                              # codec.py:14
    hm1 = A.scalar(half - 1)
    eps = A.scalar(1e-10)
    delta = np.asarray(delta, dtype=np.float32)
    amax = np.abs(delta).max(axis=-1, keepdims=True)           # codec.py:32
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = A.r(amax / hm1)                                # codec.py:33
        if dead_zone > 0.0:                                    # codec.py:36-45
            thr = A.r(amax * A.scalar(dead_zone))
            delta = np.where(np.abs(delta) < thr, np.float32(0.0), delta)
            amax_c = np.abs(delta).max(axis=-1, keepdims=True)
            amax_safe = np.where(amax_c < eps, amax, amax_c)
            scale = A.r(amax_safe / hm1)
        scale_safe = np.where(scale < eps, np.float32(1.0), scale)  # codec.py:48
        q = A.r(delta / scale_safe)                            # codec.py:50
    codes = np.rint(q)                                         # half to even
    codes = np.clip(codes, -half, half - 1)                    # codec.py:51
    codes = np.where(np.isnan(codes), 0.0, codes)              # defined NaN -> 0
    codes = np.where(scale < eps, 0.0, codes)                  # codec.py:54
    return codes.astype(np.int8), scale.astype(np.float16)    # codec.py:65


def dequantize_delta(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """codec.py:67-73: fp16(code) * fp16 scale, product rounded to fp16."""
    return (codes.astype(np.float16) * scale.astype(np.float16)).astype(np.float16)


def pack_int4_codes(codes: np.ndarray) -> np.ndarray:
    """kernels.py:34-54: nibble = clip(code+8, 0, 15); nibble i at bits 4i."""
    D = codes.shape[-1]
    W = (D + 7) // 8
    u = np.clip(codes.astype(np.int32) + 8, 0, 15).astype(np.uint32)
    if D % 8:
        pad = [(0, 0)] * (u.ndim - 1) + [(0, W * 8 - D)]
        u = np.pad(u, pad)                                     # pad nibble 0
    u = u.reshape(*codes.shape[:-1], W, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    return np.bitwise_or.reduce(u << shifts, axis=-1).astype(np.uint32)


def unpack_int4_codes(packed: np.ndarray, head_dim: int) -> np.ndarray:
    """kernels.py:57-61."""
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    e = (packed[..., None] >> shifts) & 0xF
    e = e.reshape(*packed.shape[:-1], packed.shape[-1] * 8).astype(np.int32)
    return (e[..., :head_dim] - 8).astype(np.int8)


class Component:
    """One compressed component (K or V) of ONE sequence, grown by appends.

    keyframes fp16 [H, nkf, D]; packed uint32 [H, npf, W]; scales fp16 [H, npf]
    (cache.py:46-51 without the batch axis).
    """

    def __init__(self, H: int, D: int, stride: int, delta_bits: int,
                 dead_zone: float, dtype: str = F16):
        self.H, self.D, self.stride = H, D, stride
        self.bits, self.dz, self.dtype = delta_bits, dead_zone, dtype
        W = (D + 7) // 8
        self.keyframes = np.zeros((H, 0, D), np.float16)
        self.packed = np.zeros((H, 0, W), np.uint32)
        self.scales = np.zeros((H, 0), np.float16)
        self.offset = 0

    def append(self, x: np.ndarray):
        """cache.py:87-129.  x: float32 [H, S, D] holding `dtype` values."""
        A = _Arith(self.dtype)
        kfs, pks, scs = [self.keyframes], [self.packed], [self.scales]
        new_kf = []
        n_kf0 = self.keyframes.shape[1]
        for ls in range(x.shape[1]):
            t = self.offset + ls
            tok = x[:, ls, :]
            if t % self.stride == 0:
                kf = tok.astype(np.float16)
                new_kf.append(kf)
                kfs.append(kf[:, None, :])
                continue
            g = t // self.stride
            anchor = (self.keyframes[:, g, :] if g < n_kf0 else new_kf[g - n_kf0])
            delta = A.r(tok - A.r(anchor.astype(np.float32)))      # cache.py:113
            codes, scale = quantize_delta(delta, self.bits, self.dz, self.dtype)
            pks.append(pack_int4_codes(codes)[:, None, :])
            scs.append(scale[:, 0][:, None])
        self.keyframes = np.concatenate(kfs, axis=1)
        self.packed = np.concatenate(pks, axis=1)
        self.scales = np.concatenate(scs, axis=1)
        self.offset += x.shape[1]

    def reconstruct(self) -> np.ndarray:
        """cache.py:131-156 -> fp16 [H, T, D]."""
        T = self.offset
        pos = np.arange(T)
        g = pos // self.stride
        full = self.keyframes[:, g, :]
        if self.packed.shape[1] == 0:
            return full
        pf = np.maximum(pos - g - 1, 0)
        is_p = (pos % self.stride != 0)[None, :, None]
        codes = unpack_int4_codes(self.packed, self.D)[:, pf, :]
        sc = self.scales[:, pf][..., None]
        delta = dequantize_delta(codes, sc)
        zero = np.zeros_like(delta)
        return (full + np.where(is_p, delta, zero)).astype(np.float16)


def sdpa_fallback(q: np.ndarray, rk: np.ndarray, rv: np.ndarray, scale: float,
                  causal: bool = False, mask: np.ndarray | None = None) -> np.ndarray:
    """attention.py:61-74 for fp16 inputs.  q [nq, Tq, D]; rk/rv [H, T, D];
    mask: optional boolean array [Tq, T] (attention.py:18-19)."""
    nq, Tq, D = q.shape
    H, T, _ = rk.shape
    rep = nq // H
    qs = (q.astype(np.float16) * np.float16(scale)).astype(np.float16)
    qg = qs.reshape(H, rep, Tq, D).astype(np.float64)
    s = np.einsum("hrqd,htd->hrqt", qg, rk.astype(np.float64))
    s = s.astype(np.float16).astype(np.float32)
    if causal:
        qi = np.arange(T - Tq, T)[:, None]
        ki = np.arange(T)[None, :]
        s = np.where(qi >= ki, s, np.float32(np.finfo(np.float16).min))
    if mask is not None:
        s = np.where(np.asarray(mask, bool), s, np.float32(np.finfo(np.float16).min))
    m = s.max(axis=-1, keepdims=True).astype(np.float64)
    e = np.exp(s.astype(np.float64) - m)
    w = (e / e.sum(axis=-1, keepdims=True)).astype(np.float16)
    o = np.einsum("hrqt,htd->hrqd", w.astype(np.float64), rv.astype(np.float64))
    return o.astype(np.float16).reshape(nq, Tq, D)
