"""ctypes binding of libchronoquant.so (declared in include/chronoquant.h).

The product path has no CPU fallback: if the library is missing, or no GPU
is visible when a kernel is requested, the call raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # loads the process's HIP runtime before libchronoquant.so binds to it

PKG = os.path.dirname(os.path.abspath(__file__))
# CQ_LIBRARY selects another build of the library (phase_times.py's
# diagnostic build); the product loads libchronoquant.so
LIB_PATH = os.environ.get("CQ_LIBRARY") or os.path.join(PKG, "libchronoquant.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "chronoquant.h")

CQ_OK = 0
CQ_ERR_TIMEOUT = 10
CQ_F16, CQ_BF16, CQ_F32 = 0, 1, 2
CQ_KEYS, CQ_VALUES = 0, 1
CQ_PACK_INT4, CQ_PACK_DENSE = 0, 1

_DTYPES = {torch.float16: CQ_F16, torch.bfloat16: CQ_BF16, torch.float32: CQ_F32}


class ChronoQuantError(RuntimeError):
    """A libchronoquant.so entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


class CqComponent(ctypes.Structure):
    _fields_ = [
        ("keyframes", ctypes.c_void_p),
        ("packed", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("cap_keyframes", ctypes.c_int64),
        ("cap_pframes", ctypes.c_int64),
        ("stride", ctypes.c_int32),
        ("delta_bits", ctypes.c_int32),
        ("dead_zone", ctypes.c_float),
        ("packing", ctypes.c_int32),
    ]


class CqCacheDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("k", CqComponent),
        ("v", CqComponent),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_DESC = ctypes.POINTER(CqCacheDesc)

# argtypes of every entry point declared in include/chronoquant.h
SIGNATURES = {
    "cq_quantize_delta": ([_P, _I32, _I64, _I32, _I32, _F, _P, _P, _P], _I32),
    "cq_pack_int4": ([_P, _I64, _I32, _P, _P], _I32),
    "cq_unpack_int4": ([_P, _I64, _I32, _P, _P], _I32),
    "cq_append": ([_DESC, _P, _P, _P, _P, _I32, _I64, _P, _I64, _P], _I32),
    "cq_reconstruct": ([_DESC, _I32, _I64, _P, _P], _I32),
    "cq_decode_workspace_size": ([_I32, _I32, _I32, _I32, _I64], _SZ),
    "cq_decode_attn": ([_DESC, _P, _I32, _I32, _F, _P, _I64, _I64, _P, _I32, _P, _SZ, _P], _I32),
    "cq_decode_attn_noalloc": ([_DESC, _P, _I32, _I32, _F, _P, _I64, _I64, _P, _I32, _P], _I32),
    "cq_decode_attn_generic": ([_DESC, _P, _I32, _I32, _F, _P, _I64, _I64, _P, _I32, _P, _SZ, _P], _I32),
    "cq_fp16_decode_attn": ([_P, _P, _I64, _I32, _I32, _I32, _P, _I32, _I32, _F, _P, _I64, _I64,
                             _P, _I32, _P, _SZ, _P], _I32),
    "cq_prefill_attn": ([_DESC, _P, _I32, _I32, _I64, _F, _I32, _I64, _P, _P, _SZ, _P], _I32),
    "cq_prefill_workspace_size": ([_I32, _I32, _I32, _I64, _I64], _SZ),
    "cq_gemv": ([_P, _P, _P, _I64, _I32, _I32, _P], _I32),
    "cq_gemv_rms_norm": ([_P, _P, _P, _P, _F, _P, _P, _I64, _I32, _I32, _P], _I32),
    "cq_gemv_silu": ([_P, _P, _P, _I64, _I32, _I32, _P], _I32),
    "cq_rms_norm": ([_P, _P, _P, _I64, _I32, _F, _I32, _P], _I32),
    "cq_add_rms_norm": ([_P, _P, _P, _P, _P, _I64, _I32, _F, _I32, _P], _I32),
    "cq_qkv_norm_rope": ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I64, _I32, _I32,
                          _I32, _F, _I32, _P], _I32),
    "cq_qkv_rope_append": ([_DESC, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _F, _I32, _P,
                            _I64, _P, _P], _I32),
    "cq_silu_mul": ([_P, _P, _I64, _I64, _I32, _P], _I32),
    "cq_decode_status": ([_P, _P], _I32),
    "cq_set_fold_poll_bound": ([_I32], _I32),
    "cq_status_string": ([_I32], ctypes.c_char_p),
}

_lib = None


def header_symbols() -> list[str]:
    """Names of the functions include/chronoquant.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cq_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    """Load libchronoquant.so and bind its signatures (no GPU needed)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m chronoquant_mlx_amd.build` "
            "(or __graft_entry__.build()) first")
    L = ctypes.CDLL(LIB_PATH)
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _lib = L
    return L


def status_string(status: int) -> str:
    return load().cq_status_string(int(status)).decode()


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point; raise ChronoQuantError on failure."""
    st = getattr(load(), name)(*args)
    if st != CQ_OK:
        raise ChronoQuantError(name, st, status_string(st))


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"ChronoQuant kernels support float16/bfloat16/float32, got {dt}") from None


def require_gpu(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError("ChronoQuant kernels run on the GPU only; got a CPU tensor "
                           "(there is no CPU fallback in the product path)")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_hip = None


def stream_capture_id(stream_handle: int) -> int | None:
    """Id of the stream capture in progress on a hipStream_t, None when the
    stream is not capturing.  Asks the HIP runtime the process already has
    loaded (torch's), through hipStreamGetCaptureInfo."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so", mode=os.RTLD_NOLOAD)
        _hip.hipStreamGetCaptureInfo.argtypes = [_P, ctypes.POINTER(ctypes.c_int),
                                                 ctypes.POINTER(ctypes.c_ulonglong)]
        _hip.hipStreamGetCaptureInfo.restype = ctypes.c_int
    status, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    err = _hip.hipStreamGetCaptureInfo(stream_handle, ctypes.byref(status), ctypes.byref(cid))
    if err != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed with error {err}")
    return int(cid.value) if status.value == 1 else None  # hipStreamCaptureStatusActive


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
