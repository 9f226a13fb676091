"""The C-ABI library loads and exports every symbol include/chronoquant.h
declares; argument validation answers without touching a GPU — CPU only."""
import ctypes
import subprocess

import pytest

from chronoquant_mlx_amd import _lib


def test_library_exports_every_header_symbol():
    L = _lib.load()
    names = _lib.header_symbols()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported


def test_status_strings():
    assert _lib.status_string(0) == "ok"
    for s in range(1, 11):
        assert _lib.status_string(s) != "unknown status"
    assert _lib.status_string(99) == "unknown status"


def test_validation_without_launch():
    L = _lib.load()
    # head_dim out of range, bits out of range, null pointers: rejected before any launch
    assert L.cq_quantize_delta(None, 0, 4, 300, 4, 0.0, None, None, None) == 2
    assert L.cq_quantize_delta(None, 0, 4, 128, 5, 0.0, None, None, None) == 1
    assert L.cq_quantize_delta(None, 0, 4, 128, 4, -1.0, None, None, None) == 1
    assert L.cq_quantize_delta(None, 0, 0, 128, 4, 0.0, None, None, None) == 0
    # unknown dtype code: rejected before the launch
    assert L.cq_quantize_delta(ctypes.c_void_p(8), 7, 4, 128, 4, 0.0, ctypes.c_void_p(8),
                               ctypes.c_void_p(8), None) == 3
    assert L.cq_pack_int4(None, 3, 128, None, None) == 1
    assert L.cq_unpack_int4(None, 0, 128, None, None) == 0
    d = _lib.CqCacheDesc()
    assert L.cq_append(ctypes.byref(d), None, None, None, None, 0, 1, None, 0, None) == 2
    d.batch, d.n_kv_heads, d.head_dim = 1, 8, 128
    assert L.cq_append(ctypes.byref(d), None, None, None, None, 0, 1, None, 0, None) == 1
    assert L.cq_decode_attn(None, None, 0, 8, 1.0, None, 1, 1, None, 0, None, 0, None) == 1
    assert L.cq_decode_workspace_size(0, 8, 32, 128, 100) == 0
    assert L.cq_decode_workspace_size(1, 8, 32, 128, 16384) > 0


def test_descriptor_layout_matches_header():
    # cq_component: 3 pointers, 2 int64, 3 int32 + float = 56 bytes; desc = 16 + 2*56
    assert ctypes.sizeof(_lib.CqComponent) == 56
    assert ctypes.sizeof(_lib.CqCacheDesc) == 128
    assert _lib.CqCacheDesc.k.offset == 16 and _lib.CqCacheDesc.v.offset == 72
