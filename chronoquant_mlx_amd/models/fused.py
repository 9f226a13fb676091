"""Fused elementwise ops of the end-to-end decoder, on libchronoquant.so.

They take the roles mx.fast.rms_norm, mx.fast.rope and the SwiGLU gate
play in the mlx_lm Qwen models the reference's end-to-end runs drive.
Written as torch ops, one decode step of the example decoder costs ~45
small kernels per layer and is launch-bound; each op here is one launch,
with math in fp32 and one rounding per stored value.
"""
from __future__ import annotations

import torch

from .. import _lib


def _check_weight(w: torch.Tensor, x: torch.Tensor, n: int, what: str) -> None:
    if w.dtype != x.dtype or w.numel() != n or not w.is_contiguous() or w.device != x.device:
        raise ValueError(f"{what}: weight must be a contiguous [{n}] {x.dtype} tensor on x's device")


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x @ weight.T (a bias-free torch Linear).  One input row of fp16/bf16
    (a decode step) runs cq_gemv, which streams the weight once; anything
    else runs torch's GEMM."""
    K = x.shape[-1]
    if (x.numel() != K or x.dtype not in (torch.float16, torch.bfloat16)
            or weight.dtype != x.dtype or K % 8 or not weight.is_contiguous()
            or weight.data_ptr() % 16 or x.device != weight.device or x.device.type != "cuda"):
        return torch.nn.functional.linear(x, weight)
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    N = weight.shape[0]
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    _lib.call("cq_gemv", weight.data_ptr(), x.data_ptr(), y.data_ptr(), N, K,
              _lib.dtype_code(x.dtype), _lib.stream_of(x))
    return y


def _one_row_ok(x: torch.Tensor, weight: torch.Tensor, k: int) -> bool:
    return (x.numel() == k and x.dtype in (torch.float16, torch.bfloat16) and weight.dtype == x.dtype
            and k % 8 == 0 and weight.is_contiguous() and weight.data_ptr() % 16 == 0
            and x.is_contiguous() and x.data_ptr() % 16 == 0 and x.device == weight.device
            and x.device.type == "cuda")


def linear_rms_norm(x: torch.Tensor, residual: torch.Tensor | None, norm_weight: torch.Tensor,
                    eps: float, weight: torch.Tensor, want_h: bool = False):
    """One row: h = x + residual (or x), y = rms_norm(h, norm_weight) @ weight.T
    in one launch (cq_gemv_rms_norm).  Returns (y, h) with h None unless
    want_h (which needs a residual)."""
    K = x.shape[-1]
    ok = (_one_row_ok(x, weight, K) and K <= 8192 and norm_weight.dtype == x.dtype
          and norm_weight.is_contiguous() and norm_weight.data_ptr() % 16 == 0
          and (residual is None or (residual.is_contiguous() and residual.dtype == x.dtype
                                    and residual.numel() == K and residual.data_ptr() % 16 == 0)))
    if not ok:
        h = x if residual is None else None
        if residual is not None:
            h, xn = add_rms_norm(x, residual, norm_weight, eps)
        else:
            xn = rms_norm(x, norm_weight, eps)
        return linear(xn, weight), (h if want_h else None)
    if want_h and residual is None:
        raise ValueError("linear_rms_norm: want_h needs a residual")
    N = weight.shape[0]
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    h = torch.empty_like(x) if want_h else None
    _lib.call("cq_gemv_rms_norm", weight.data_ptr(), x.data_ptr(),
              None if residual is None else residual.data_ptr(), norm_weight.data_ptr(),
              float(eps), None if h is None else h.data_ptr(), y.data_ptr(), N, K,
              _lib.dtype_code(x.dtype), _lib.stream_of(x))
    return y, h


def linear_silu(gu: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """One row: silu_mul(gu) @ weight.T in one launch (cq_gemv_silu)."""
    K = gu.shape[-1] // 2
    if not (_one_row_ok(gu.reshape(-1)[:K], weight, K) and gu.numel() == 2 * K
            and gu.is_contiguous()):
        return linear(silu_mul(gu), weight)
    N = weight.shape[0]
    y = torch.empty(*gu.shape[:-1], N, dtype=gu.dtype, device=gu.device)
    _lib.call("cq_gemv_silu", weight.data_ptr(), gu.data_ptr(), y.data_ptr(), N, K,
              _lib.dtype_code(gu.dtype), _lib.stream_of(gu))
    return y


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2, -1) + eps) * weight over the last dim."""
    _lib.require_gpu(x)
    x = x.contiguous()
    dim = x.shape[-1]
    _check_weight(weight, x, dim, "rms_norm")
    y = torch.empty_like(x)
    _lib.call("cq_rms_norm", x.data_ptr(), weight.data_ptr(), y.data_ptr(), x.numel() // dim, dim,
              float(eps), _lib.dtype_code(x.dtype), _lib.stream_of(x))
    return y


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """h = x + residual (rounded to the dtype), y = rms_norm(h); returns (h, y)."""
    _lib.require_gpu(x)
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError("add_rms_norm: residual must match x's shape and dtype")
    x, residual = x.contiguous(), residual.contiguous()
    dim = x.shape[-1]
    _check_weight(weight, x, dim, "add_rms_norm")
    h, y = torch.empty_like(x), torch.empty_like(x)
    _lib.call("cq_add_rms_norm", x.data_ptr(), residual.data_ptr(), weight.data_ptr(),
              h.data_ptr(), y.data_ptr(), x.numel() // dim, dim, float(eps),
              _lib.dtype_code(x.dtype), _lib.stream_of(x))
    return h, y


def qkv_norm_rope(qkv: torch.Tensor, n_q_heads: int, n_kv_heads: int,
                  q_weight: torch.Tensor | None, k_weight: torch.Tensor | None,
                  cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                  eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused QKV projection output [B, L, (nq + 2 nkv) * 128] -> q [B, nq, L,
    128], k and v [B, nkv, L, 128]: q/k heads RMSNorm'd (weight None: none)
    and rotated at `positions` ([L] or [B, L]) with the fp32 tables cos/sin
    [max_pos, 64]; v heads copied.  A position outside the tables gives NaN."""
    _lib.require_gpu(qkv)
    B, L, W = qkv.shape
    D = 128
    if W != (n_q_heads + 2 * n_kv_heads) * D:
        raise ValueError("qkv_norm_rope: last dim must be (n_q_heads + 2 n_kv_heads) * 128")
    qkv = qkv.contiguous()
    for t in (cos, sin):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != D // 2 or t.device != qkv.device:
            raise ValueError("qkv_norm_rope: cos/sin must be fp32 [max_pos, 64] on qkv's device")
    cos, sin = cos.contiguous(), sin.contiguous()
    for w, what in ((q_weight, "q"), (k_weight, "k")):
        if w is not None:
            _check_weight(w, qkv, D, f"qkv_norm_rope ({what} norm)")
    positions = positions.to(device=qkv.device, dtype=torch.int64)
    if positions.dim() == 1 and positions.numel() == L:
        bstride = 0
    elif positions.shape == (B, L):
        bstride = L
    else:
        raise ValueError("qkv_norm_rope: positions must be [L] or [B, L]")
    positions = positions.contiguous()
    q = torch.empty(B, n_q_heads, L, D, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty(B, n_kv_heads, L, D, dtype=qkv.dtype, device=qkv.device)
    v = torch.empty_like(k)
    _lib.call("cq_qkv_norm_rope", qkv.data_ptr(), _lib.ptr(q_weight), _lib.ptr(k_weight),
              q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(),
              cos.shape[0], positions.data_ptr(), bstride, B, L, n_q_heads, n_kv_heads, D,
              float(eps), _lib.dtype_code(qkv.dtype), _lib.stream_of(qkv))
    return q, k, v


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate_up[..., :n]) * gate_up[..., n:] for a fused [gate | up] projection."""
    _lib.require_gpu(gate_up)
    gate_up = gate_up.contiguous()
    n = gate_up.shape[-1] // 2
    if gate_up.shape[-1] != 2 * n:
        raise ValueError("silu_mul: last dim must be even")
    y = torch.empty(*gate_up.shape[:-1], n, dtype=gate_up.dtype, device=gate_up.device)
    _lib.call("cq_silu_mul", gate_up.data_ptr(), y.data_ptr(), gate_up.numel() // (2 * n), n,
              _lib.dtype_code(gate_up.dtype), _lib.stream_of(gate_up))
    return y
