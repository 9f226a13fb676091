"""ChronoQuant residual codec on the GPU.

Mirrors ChronoQuantCodecMLX (reference codec.py:4-73): symmetric per-row
residual quantisation with an optional dead zone.  quantize_delta runs the
gfx950 codec kernel (one wavefront per row, DPP absmax) through
cq_quantize_delta; the cache's append path runs the same device code fused
with packing, so this object is the standalone operator and the holder of
the codec parameters.
"""
from __future__ import annotations

import torch

from . import _lib


class ChronoQuantCodec:
    """Symmetric delta quantisation with dead-zone support (codec.py:4-21).

    half_levels = 2**delta_bits // 2; codes lie in [-half_levels,
    half_levels - 1]; delta_bits must be 2, 3 or 4 (codes live in INT4 lanes).
    """

    def __init__(self, stride: int = 32, delta_bits: int = 4, dead_zone_ratio: float = 0.0,
                 log_interval: int = 100):
        if delta_bits not in (2, 3, 4):
            raise ValueError(f"delta_bits must be 2, 3 or 4 (INT4 lanes), got {delta_bits}")
        if dead_zone_ratio < 0:
            raise ValueError("dead_zone_ratio must be >= 0")
        self.stride = stride
        self.delta_bits = delta_bits
        self.half_levels = (2 ** delta_bits) // 2
        self.dead_zone_ratio = dead_zone_ratio
        # distribution logging (codec.py:17-21, 56-63); 0 disables it
        self._total_elements = 0
        self._zero_elements = 0
        self._log_interval = log_interval
        self._call_count = 0

    def quantize_delta(self, delta: torch.Tensor):
        """codec.py:23-65.  delta [..., D] (fp16/bf16/fp32, GPU) ->
        (codes int8 [..., D], scales fp16 [..., 1])."""
        _lib.require_gpu(delta)
        delta = delta.contiguous()
        D = delta.shape[-1]
        rows = delta.numel() // D if D else 0
        codes = torch.empty(delta.shape, dtype=torch.int8, device=delta.device)
        scales = torch.empty(*delta.shape[:-1], 1, dtype=torch.float16, device=delta.device)
        _lib.call("cq_quantize_delta", delta.data_ptr(), _lib.dtype_code(delta.dtype), rows, D,
                  self.delta_bits, float(self.dead_zone_ratio), codes.data_ptr(),
                  scales.data_ptr(), _lib.stream_of(delta))
        # every _log_interval-th call: the share of zero codes in this call
        # (a host sync, as the reference's counter does)
        self._call_count += 1
        if self._log_interval and self._call_count % self._log_interval == 0:
            zeros = int((codes == 0).sum().item())
            self._total_elements += codes.numel()
            self._zero_elements += zeros
            print(f"  [codec] {self.delta_bits}-bit residuals, dead zone "
                  f"{self.dead_zone_ratio:.2f}: {zeros / max(codes.numel(), 1):.1%} of "
                  f"{codes.numel()} codes are zero")
        return codes, scales

    def dequantize_delta(self, codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """codec.py:67-73: fp16(code) * fp16 scale, rounded to fp16."""
        return codes.to(torch.float16) * scale.to(torch.float16)


# the reference's class name
ChronoQuantCodecMLX = ChronoQuantCodec
