"""Synthetic decode workloads of the benchmark configurations.

K and V are independent fp16 AR(1) streams per (sequence, kv head, channel):
x_0 ~ N(0, noise^2/(1-rho^2)) (stationary), x_t = rho*x_{t-1} + noise*N(0,1),
scaled by a per-channel sigma ~ LogNormal(0, 0.5); a fraction of the
(kv head, channel) pairs of each sequence may be outliers at 8x sigma.
Queries are fp16 N(0, 1).  numpy PCG64 with fixed seeds, float64 math, one
rounding to fp16 at the end.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_K, SEED_V, SEED_Q, SEED_SIGMA = 1000, 2000, 3000, 4000


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    B: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    T: int                      # context length (max length when ragged)
    stride_k: int
    stride_v: int
    delta_bits_k: int = 4
    delta_bits_v: int = 4
    dead_zone_k: float = 0.0
    dead_zone_v: float = 0.0
    outlier_frac: float = 0.0
    ragged_min: int = 0         # > 0: lengths ~ U{ragged_min..T}
    rho: float = 0.98
    noise: float = 0.2
    extra: dict = field(default_factory=dict)

    def lengths(self, seed: int = 5000) -> np.ndarray:
        if self.ragged_min <= 0:
            return np.full(self.B, self.T, np.int64)
        rng = np.random.default_rng(seed)
        return rng.integers(self.ragged_min, self.T + 1, size=self.B).astype(np.int64)


# BASELINE.json configs[0..3]
CONFIGS = {
    "c0": DecodeConfig("c0", B=1, n_q_heads=8, n_kv_heads=8, head_dim=128, T=4096,
                       stride_k=32, stride_v=8),
    "c1": DecodeConfig("c1", B=1, n_q_heads=32, n_kv_heads=8, head_dim=128, T=16384,
                       stride_k=32, stride_v=8),
    "c2": DecodeConfig("c2", B=8, n_q_heads=32, n_kv_heads=8, head_dim=128, T=32768,
                       stride_k=64, stride_v=32, delta_bits_k=4, delta_bits_v=3,
                       dead_zone_k=0.0, dead_zone_v=0.05, outlier_frac=0.01),
    "c3": DecodeConfig("c3", B=32, n_q_heads=32, n_kv_heads=8, head_dim=128, T=32768,
                       stride_k=32, stride_v=8, dead_zone_v=0.05, ragged_min=1024),
    # the north star's target shape: configs[1]'s GQA 32/8 @16K with Full-Throttle V3
    "ftv3_16k": DecodeConfig("ftv3_16k", B=1, n_q_heads=32, n_kv_heads=8, head_dim=128,
                             T=16384, stride_k=64, stride_v=32, delta_bits_k=4,
                             delta_bits_v=3, dead_zone_k=0.0, dead_zone_v=0.05,
                             outlier_frac=0.01),
}


def sigmas(B: int, H: int, D: int, outlier_frac: float, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    sig = rng.lognormal(0.0, 0.5, size=(B, H, D))
    n_out = int(round(outlier_frac * H * D))
    for b in range(B):
        if n_out:
            idx = rng.permutation(H * D)[:n_out]
            sig[b].reshape(-1)[idx] *= 8.0
    return sig


def ar1_stream(B: int, H: int, T: int, D: int, seed: int, sigma: np.ndarray,
               rho: float = 0.98, noise: float = 0.2) -> np.ndarray:
    """fp16 [B, H, T, D] AR(1) stream."""
    rng = np.random.default_rng(seed)
    out = np.empty((B, H, T, D), np.float16)
    x = rng.normal(0.0, noise / np.sqrt(1.0 - rho * rho), size=(B, H, D))
    out[:, :, 0] = (sigma * x).astype(np.float16)
    for t in range(1, T):
        x = rho * x + noise * rng.standard_normal((B, H, D))
        out[:, :, t] = (sigma * x).astype(np.float16)
    return out


def make_kv(cfg: DecodeConfig, T: int | None = None, B: int | None = None, layer: int = 0):
    """(K, V) fp16 [B, H, T, D] for the config (optionally truncated)."""
    T = cfg.T if T is None else T
    B = cfg.B if B is None else B
    H, D = cfg.n_kv_heads, cfg.head_dim
    sk = sigmas(B, H, D, cfg.outlier_frac, SEED_SIGMA + layer)
    sv = sigmas(B, H, D, cfg.outlier_frac, SEED_SIGMA + 100 + layer)
    k = ar1_stream(B, H, T, D, SEED_K + layer, sk, cfg.rho, cfg.noise)
    v = ar1_stream(B, H, T, D, SEED_V + layer, sv, cfg.rho, cfg.noise)
    return k, v


def make_q(cfg: DecodeConfig, B: int | None = None, seed: int = SEED_Q) -> np.ndarray:
    B = cfg.B if B is None else B
    rng = np.random.default_rng(seed)
    return rng.standard_normal((B, cfg.n_q_heads, cfg.head_dim)).astype(np.float16)


def compressed_bytes(T: int, H: int, D: int, stride_k: int, stride_v: int) -> int:
    """Active bytes of one sequence's cache (the reference's nbytes,
    cache.py:274-287): I-frames fp16 + packed rows + fp16 scales, K and V."""
    W = (D + 7) // 8
    total = 0
    for s in (stride_k, stride_v):
        nkf = 0 if T <= 0 else (T - 1) // s + 1
        npf = T - nkf
        total += H * nkf * D * 2 + H * npf * (W * 4 + 2)
    return total


def algorithmic_decode_bytes(cfg: DecodeConfig, lengths=None) -> int:
    """Bytes one decode step must move: compressed cache + Q + O (fp16)."""
    lengths = cfg.lengths() if lengths is None else lengths
    cache = sum(compressed_bytes(int(T), cfg.n_kv_heads, cfg.head_dim, cfg.stride_k,
                                 cfg.stride_v) for T in lengths)
    return cache + 2 * len(lengths) * cfg.n_q_heads * cfg.head_dim * 2


def make_kv_device(cfg: DecodeConfig, T: int, B: int, device, seed: int = 7000):
    """(K, V) fp16 [B, H, T, D] with the same AR(1) statistics, generated on
    the GPU (torch Philox) for workloads too large for the host generator.
    The recurrence is evaluated in 256-token chunks in closed form:
    x_{t+i} = rho^(i+1) x_{t-1} + sum_{j<=i} rho^(i-j) e_j."""
    import torch
    H, D = cfg.n_kv_heads, cfg.head_dim
    rho, noise, L = cfg.rho, cfg.noise, 256
    j = torch.arange(L, device=device, dtype=torch.float64)
    pw = (rho ** (j + 1)).float()[:, None]
    fwd = (rho ** j).float()[:, None]
    inv = (rho ** (-j)).float()[:, None]
    outs = []
    for comp in range(2):
        g = torch.Generator(device=device)
        g.manual_seed(seed + comp)
        sig = torch.exp(0.5 * torch.randn(B, H, D, generator=g, device=device))
        n_out = int(round(cfg.outlier_frac * H * D))
        if n_out:
            for b in range(B):
                idx = torch.randperm(H * D, generator=g, device=device)[:n_out]
                sig[b].view(-1)[idx] *= 8.0
        out = torch.empty(B, H, T, D, dtype=torch.float16, device=device)
        x = torch.randn(B, H, 1, D, generator=g, device=device) * (noise / (1.0 - rho * rho) ** 0.5)
        out[:, :, :1] = (sig[:, :, None, :] * x).half()
        t = 1
        while t < T:
            n = min(L, T - t)
            eps = torch.randn(B, H, n, D, generator=g, device=device) * noise
            xs = pw[:n] * x + fwd[:n] * torch.cumsum(eps * inv[:n], dim=2)
            out[:, :, t:t + n] = (sig[:, :, None, :] * xs).half()
            x = xs[:, :, n - 1:n]
            t += n
        outs.append(out)
    return outs[0], outs[1]
