"""ctypes front end of the C oracle (oracle/libcq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  Each wrapper names the reference lines the C
function restates (see the header of oracle/cq_oracle.c).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcq_oracle.so")

DT = {"f16": 0, "bf16": 1, "f32": 2}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.cqo_quantize_delta.argtypes = [I32, P, I64, I32, I32, F, P, P]
        L.cqo_pack_int4.argtypes = [P, I64, I32, P]
        L.cqo_unpack_int4.argtypes = [P, I64, I32, P]
        L.cqo_append_component.argtypes = [I32, P, I64, I64, I32, I32, I64, I64, I32,
                                           I32, F, P, I64, P, I64, P]
        L.cqo_append_component.restype = I32
        L.cqo_reconstruct_component.argtypes = [I32, I32, I64, I32, P, I64, P, I64, P, P]
        L.cqo_sdpa_fallback.argtypes = [P, P, P, I32, I32, I64, I64, I32, F, I32, P]
        L.cqo_sdpa_fallback_mask.argtypes = [P, P, P, I32, I32, I64, I64, I32, F, I32, P, P]
        L.cqo_sdpa_fallback_bf16q.argtypes = [P, P, P, I32, I32, I64, I64, I32, F, I32, P, P]
        L.cqo_sdpa_fused.argtypes = [P, I32, I32, I32, I64, F, I32, I32,
                                     P, I64, P, I64, P, P, I64, P, I64, P, P]
        L.cqo_sdpa_fused_absw.argtypes = [P, I32, I32, I32, I64, F, I32, I32,
                                          P, I64, P, I64, P, P, I64, P, I64, P, P, P]
        L.cqo_sdpa_exact.argtypes = [P, P, P, I32, I32, I64, I32, ctypes.c_double, P]
        L.cqo_decode_step.argtypes = [P, I32, I32, I32, I64, F, I32, I32,
                                      P, I64, P, I64, P, P, I64, P, I64, P, P, P, P]
        L.cqo_threads.restype = I32
        L.cqo_set_threads.argtypes = [I32]
        L.cqo_f32_to_f16_array.argtypes = [P, I64, P]
        L.cqo_f16_to_f32_array.argtypes = [P, I64, P]
        L.cqo_f32_to_bf16_array.argtypes = [P, I64, P]
        L.cqo_num_keyframes.argtypes = [I64, I32]
        L.cqo_num_keyframes.restype = I64
        L.cqo_num_pframes.argtypes = [I64, I32]
        L.cqo_num_pframes.restype = I64
        L.cqb_fused_decode_f32.argtypes = [P, I32, I32, I32, I64, F, I32, I32,
                                           P, I64, P, I64, P, P, I64, P, I64, P, I32, P]
        L.cqb_fused_decode_f32.restype = I32
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """Input values as the raw storage the C oracle reads for `dtype`."""
    if dtype == "f16":
        return np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    if dtype == "bf16":
        if x.dtype == np.uint16:
            return np.ascontiguousarray(x)
        return f32_to_bf16(np.asarray(x, np.float32))
    return np.ascontiguousarray(x, dtype=np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().cqo_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().cqo_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().cqo_f32_to_bf16_array(_p(x), x.size, _p(out))
    return out


def quantize_delta(delta: np.ndarray, delta_bits: int, dead_zone: float,
                   dtype: str = "f16"):
    """codec.py:23-65.  delta [..., D] -> (int8 codes [..., D], fp16 scales [...])."""
    D = delta.shape[-1]
    raw = _bits(delta, dtype)
    n = raw.size // D
    codes = np.empty(raw.shape, np.int8)
    scales = np.empty(raw.shape[:-1], np.uint16)
    lib().cqo_quantize_delta(DT[dtype], _p(raw), n, D, delta_bits, float(dead_zone),
                             _p(codes), _p(scales))
    return codes, scales.view(np.float16)


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """kernels.py:34-54."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    D = codes.shape[-1]
    W = (D + 7) // 8
    out = np.empty(codes.shape[:-1] + (W,), np.uint32)
    lib().cqo_pack_int4(_p(codes), codes.size // D, D, _p(out))
    return out


def unpack_int4(packed: np.ndarray, head_dim: int) -> np.ndarray:
    """kernels.py:57-61."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    W = packed.shape[-1]
    n = packed.size // W
    out = np.empty(packed.shape[:-1] + (head_dim,), np.int8)
    lib().cqo_unpack_int4(_p(packed), n, head_dim, _p(out))
    return out


def num_keyframes(n: int, stride: int) -> int:
    return int(lib().cqo_num_keyframes(n, stride))


def num_pframes(n: int, stride: int) -> int:
    return int(lib().cqo_num_pframes(n, stride))


class OracleComponent:
    """One component (K or V) of one sequence, stored at fixed capacity.

    keyframes fp16 [H, cap_kf, D], packed uint32 [H, cap_pf, W], scales fp16
    [H, cap_pf]; `active()` returns the reference's tensors (cache.py:63-85).
    """

    def __init__(self, H, D, stride, delta_bits, dead_zone, capacity):
        self.H, self.D, self.stride = H, D, stride
        self.bits, self.dz = delta_bits, dead_zone
        self.W = (D + 7) // 8
        self.cap_kf = max(1, num_keyframes(capacity, stride))
        self.cap_pf = max(1, num_pframes(capacity, stride))
        self.kf = np.zeros((H, self.cap_kf, D), np.uint16)
        self.pk = np.zeros((H, self.cap_pf, self.W), np.uint32)
        self.sc = np.zeros((H, self.cap_pf), np.uint16)
        self.offset = 0

    def append(self, x: np.ndarray, dtype: str = "f16"):
        """cache.py:87-129.  x [H, S, D] values of `dtype`."""
        raw = _bits(x, dtype)
        H, S, D = raw.shape
        rc = lib().cqo_append_component(DT[dtype], _p(raw), S * D, D, H, D, S,
                                        self.offset, self.stride, self.bits,
                                        float(self.dz), _p(self.kf), self.cap_kf,
                                        _p(self.pk), self.cap_pf, _p(self.sc))
        if rc != 0:
            raise ValueError("oracle capacity exceeded")
        self.offset += S

    def active(self):
        nkf = num_keyframes(self.offset, self.stride)
        npf = num_pframes(self.offset, self.stride)
        return (self.kf[:, :nkf].view(np.float16), self.pk[:, :npf],
                self.sc[:, :npf].view(np.float16))

    def reconstruct(self) -> np.ndarray:
        """cache.py:131-156 -> fp16 [H, T, D]."""
        T = self.offset
        out = np.empty((self.H, T, self.D), np.uint16)
        lib().cqo_reconstruct_component(self.H, self.D, T, self.stride, _p(self.kf),
                                        self.cap_kf, _p(self.pk), self.cap_pf,
                                        _p(self.sc), _p(out))
        return out.view(np.float16)


def sdpa_fallback(q: np.ndarray, rk: np.ndarray, rv: np.ndarray, scale: float,
                  causal: bool = False, mask: np.ndarray | None = None) -> np.ndarray:
    """attention.py:61-74.  q fp16 [nq, Tq, D]; rk, rv fp16 [H, T, D]; mask:
    optional boolean array [Tq, T] (attention.py:18-19), on top of causal."""
    q = np.ascontiguousarray(q, np.float16).view(np.uint16)
    rk = np.ascontiguousarray(rk, np.float16).view(np.uint16)
    rv = np.ascontiguousarray(rv, np.float16).view(np.uint16)
    nq, Tq, D = q.shape
    H, T, _ = rk.shape
    out = np.empty((nq, Tq, D), np.uint16)
    if mask is None:
        lib().cqo_sdpa_fallback(_p(q), _p(rk), _p(rv), nq, H, Tq, T, D, float(scale),
                                int(causal), _p(out))
    else:
        m = np.ascontiguousarray(np.broadcast_to(np.asarray(mask, bool), (Tq, T)), np.uint8)
        lib().cqo_sdpa_fallback_mask(_p(q), _p(rk), _p(rv), nq, H, Tq, T, D, float(scale),
                                     int(causal), _p(m), _p(out))
    return out.view(np.float16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def sdpa_fallback_bf16q(q_bits: np.ndarray, rk: np.ndarray, rv: np.ndarray, scale: float,
                        causal: bool = False, mask: np.ndarray | None = None) -> np.ndarray:
    """attention.py:61-74 with bf16 queries (MLX's bf16 x fp16 promotion:
    fp32 scores and weights, bf16 output).  q_bits: bf16 bit patterns
    [nq, Tq, D]; rk, rv fp16 [H, T, D].  Returns bf16 bit patterns."""
    q = np.ascontiguousarray(q_bits, np.uint16)
    rk = np.ascontiguousarray(rk, np.float16).view(np.uint16)
    rv = np.ascontiguousarray(rv, np.float16).view(np.uint16)
    nq, Tq, D = q.shape
    H, T, _ = rk.shape
    out = np.empty((nq, Tq, D), np.uint16)
    m = None
    if mask is not None:
        m = np.ascontiguousarray(np.broadcast_to(np.asarray(mask, bool), (Tq, T)), np.uint8)
    lib().cqo_sdpa_fallback_bf16q(_p(q), _p(rk), _p(rv), nq, H, Tq, T, D, float(scale),
                                  int(causal), None if m is None else _p(m), _p(out))
    return out


def sdpa_fused(q: np.ndarray, ck: OracleComponent, cv: OracleComponent,
               scale: float, T: int | None = None, return_absw: bool = False):
    """MSL kernels.py:79-228 semantics over the first T tokens (default: all
    appended).  q fp16 [nq, D] -> fp32 [nq, D]; with return_absw also the
    softmax-weighted mean of |v| per element, (out, absw)."""
    q = np.ascontiguousarray(q, np.float16).view(np.uint16)
    nq, D = q.shape
    T = ck.offset if T is None else int(T)
    assert 0 < T <= min(ck.offset, cv.offset)
    out = np.empty((nq, D), np.float32)
    absw = np.empty((nq, D), np.float32) if return_absw else None
    lib().cqo_sdpa_fused_absw(_p(q), nq, ck.H, D, T, float(scale), ck.stride,
                              cv.stride, _p(ck.kf), ck.cap_kf, _p(ck.pk), ck.cap_pf,
                              _p(ck.sc), _p(cv.kf), cv.cap_kf, _p(cv.pk), cv.cap_pf,
                              _p(cv.sc), _p(out), None if absw is None else _p(absw))
    return (out, absw) if return_absw else out


def fused_decode_f32(q: np.ndarray, ck: OracleComponent, cv: OracleComponent,
                     scale: float, T: int | None = None, n_chunks: int = 0) -> np.ndarray:
    """CPU baseline (oracle/cq_cpu_baseline.c) of the fused operator
    kernels.py:79-228 in fp32: blockwise online softmax over key chunks on
    OpenMP threads.  q fp16 [nq, D] -> fp32 [nq, D]."""
    q = np.ascontiguousarray(q, np.float16).view(np.uint16)
    nq, D = q.shape
    T = ck.offset if T is None else int(T)
    assert 0 <= T <= min(ck.offset, cv.offset)
    out = np.empty((nq, D), np.float32)
    rc = lib().cqb_fused_decode_f32(_p(q), nq, ck.H, D, T, float(scale), ck.stride,
                                    cv.stride, _p(ck.kf), ck.cap_kf, _p(ck.pk), ck.cap_pf,
                                    _p(ck.sc), _p(cv.kf), cv.cap_kf, _p(cv.pk), cv.cap_pf,
                                    _p(cv.sc), int(n_chunks), _p(out))
    if rc != 0:
        raise ValueError("shape outside the CPU baseline's vectorised form")
    return out


def sdpa_exact(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Binary64 softmax attention.  q fp16 [nq, D]; k, v fp16 [H, T, D]."""
    q = np.ascontiguousarray(q, np.float16).view(np.uint16)
    k = np.ascontiguousarray(k, np.float16).view(np.uint16)
    v = np.ascontiguousarray(v, np.float16).view(np.uint16)
    nq, D = q.shape
    H, T, _ = k.shape
    out = np.empty((nq, D), np.float64)
    lib().cqo_sdpa_exact(_p(q), _p(k), _p(v), nq, H, T, D, float(scale), _p(out))
    return out


def decode_step(q: np.ndarray, ck: OracleComponent, cv: OracleComponent,
                scale: float, scratch=None) -> np.ndarray:
    """Reference per-layer decode work (cache.py:131-160 + attention.py:61-74)."""
    q = np.ascontiguousarray(q, np.float16).view(np.uint16)
    nq, D = q.shape
    T = ck.offset
    if scratch is None:
        scratch = (np.empty((ck.H, T, D), np.uint16), np.empty((cv.H, T, D), np.uint16))
    rk, rv = scratch
    out = np.empty((nq, D), np.uint16)
    lib().cqo_decode_step(_p(q), nq, ck.H, D, T, float(scale), ck.stride, cv.stride,
                          _p(ck.kf), ck.cap_kf, _p(ck.pk), ck.cap_pf, _p(ck.sc),
                          _p(cv.kf), cv.cap_kf, _p(cv.pk), cv.cap_pf, _p(cv.sc),
                          _p(rk), _p(rv), _p(out))
    return out.view(np.float16)


def threads() -> int:
    return int(lib().cqo_threads())


def set_threads(n: int) -> None:
    lib().cqo_set_threads(int(n))
