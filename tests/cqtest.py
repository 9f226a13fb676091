"""Shared helpers of the GPU parity tests: build the same cache on the GPU
(through libchronoquant.so) and in the CPU oracle, and compare."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

# Decode parity bar of the BASELINE north star, read as the usual (atol, rtol)
# pair: |got - ref| <= ATOL + RTOL * |ref| elementwise against the oracle's
# restatement of the reference's reconstruct-fallback path.  (At c2 the
# outputs reach +-3.5 where one fp16 ulp is 1.95e-3; the fallback itself is
# 2.5e-3 max-abs away from binary64 attention on the same reconstruction.)
ATOL, RTOL = 2e-3, 1e-2
# Tight bar against the restatement of the reference's fused-kernel semantics
# (fp32 dequant, no fp16 rounding of scores or weights).  Portable kernel: one
# fp16 output rounding (2^-12 relative) plus fp32 accumulation.  MFMA kernel:
# additionally its P.V operands carry the softmax weights p and p*s in fp16
# (<= 2^-12 relative per weight, the rounding point the reference's fallback
# also has, attention.py:72); at c2 (8x outlier channels) that reaches
# ~2.6e-4 absolute where the output nearly cancels.
TIGHT_ATOL, TIGHT_RTOL = 2e-4, 1e-3
TIGHT_ATOL_MFMA, TIGHT_RTOL_MFMA = 5e-4, 2e-3


def to_gpu(x: np.ndarray, dtype=torch.float16) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def build_gpu_cache(k: np.ndarray, v: np.ndarray, *, stride_k, stride_v, bits_k=4, bits_v=4,
                    dz_k=0.0, dz_v=0.0, chunks=None, dtype=torch.float16):
    """ChronoQuantCache filled with fp16 k, v [B, H, T, D] (appended in chunks)."""
    from chronoquant_mlx_amd import ChronoQuantCache
    cache = ChronoQuantCache(stride_k=stride_k, stride_v=stride_v, delta_bits_k=bits_k,
                             delta_bits_v=bits_v, dead_zone_k=dz_k, dead_zone_v=dz_v)
    T = k.shape[2]
    kt, vt = to_gpu(k, dtype), to_gpu(v, dtype)
    if chunks is None:
        chunks = [T]
    pos = 0
    for S in chunks:
        cache.update_and_fetch(kt[:, :, pos: pos + S], vt[:, :, pos: pos + S])
        pos += S
    assert pos == T
    return cache


def build_oracle(k_b: np.ndarray, v_b: np.ndarray, *, stride_k, stride_v, bits_k=4, bits_v=4,
                 dz_k=0.0, dz_v=0.0, dtype="f16"):
    """Oracle components of ONE sequence (k_b, v_b [H, T, D])."""
    H, T, D = k_b.shape
    ck = O.OracleComponent(H, D, stride_k, bits_k, dz_k, capacity=T)
    cv = O.OracleComponent(H, D, stride_v, bits_v, dz_v, capacity=T)
    ck.append(k_b, dtype)
    cv.append(v_b, dtype)
    return ck, cv


def assert_state_equal(cache, b: int, ck, cv):
    """GPU cache state of sequence b == oracle state, bit for bit."""
    st = cache.state
    for i, comp in ((0, ck), (1, cv)):
        kf, pk, sc = comp.active()
        g_kf = st[i][b].cpu().numpy()
        g_pk = st[2 + 2 * i][b].cpu().numpy()
        g_sc = st[3 + 2 * i][b].cpu().numpy()
        assert np.array_equal(g_kf.view(np.uint16), kf.view(np.uint16)), f"keyframes[{i}] differ"
        diff = np.argwhere(g_pk != pk)
        assert diff.size == 0, f"packed[{i}] differ at {diff[:5].tolist()} ({len(diff)} words)"
        assert np.array_equal(g_sc.view(np.uint16), sc.view(np.uint16)), f"scales[{i}] differ"


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    """Elementwise |got - ref| <= atol + rtol*|ref|, and relative L2 <= rtol."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert np.all(err <= bound), (f"{what}: |d|={err[worst]:.3e} > {bound[worst]:.3e} at "
                                  f"{tuple(int(i) for i in worst)} (ref {ref[worst]:.4f}); "
                                  f"max-abs {err.max():.3e}")
    assert rel <= rtol, f"{what} rel {rel:.3e} > {rtol}"
    return float(err.max()), float(rel)


def assert_close_fallback(got, fb, exact, what=""):
    """The fallback bar where the fallback's own rounding is large (c2's 8x
    outlier channels): |got - fb| <= ATOL + RTOL*|fb| + |fb - exact|
    elementwise, exact = binary64 attention over the same fp16
    reconstruction, and relative L2 to the fallback <= RTOL.  The reference's
    own fused kernel (kernels.py:79-228: fp32 dequant, fp32 scores) differs
    from its fallback (fp16 reconstruction, fp16 scores and weights) by more
    than ATOL + RTOL*|fb| on some c2 elements; both stay within the bar of
    exact attention, so the fallback's distance to it is the slack."""
    got = np.asarray(got, np.float64)
    fb = np.asarray(fb, np.float64)
    slack = np.abs(fb - np.asarray(exact, np.float64))
    err = np.abs(got - fb)
    bound = ATOL + RTOL * np.abs(fb) + slack
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    rel = np.linalg.norm(got - fb) / max(np.linalg.norm(fb), 1e-30)
    assert np.all(err <= bound), (f"{what}: |d|={err[worst]:.3e} > {bound[worst]:.3e} at "
                                  f"{tuple(int(i) for i in worst)} (fallback {fb[worst]:.4f}, "
                                  f"its own error {slack[worst]:.3e})")
    assert rel <= RTOL, f"{what} rel {rel:.3e} > {RTOL}"
    return float(err.max()), float(rel)


# With the softmax-weighted mean of |v| (absw, oracle.sdpa_fused) the MFMA
# kernel's tight bar takes absw in place of |ref| in its relative part:
# weights p and p*s_v carried in fp16 (relative error 2^-11 each) move a
# weighted mean of v by a multiple of 2^-11 * absw, which is not small
# against |ref| where the output cancels (c2's 8x outlier channels:
# |ref| << absw).  The absolute part stays TIGHT_ATOL_MFMA: weights below
# fp16's normal range carry an absolute error up to 2^-25 each, which over
# tens of thousands of tokens no relative term bounds.  absw >= |ref|, so
# elsewhere this is the |ref| bar.
TIGHT_ATOL_ABSW, TIGHT_U_ABSW = 5e-4, 2.0 ** -9


def assert_tight(got, ref, what="", mfma=True, absw=None):
    if mfma and absw is not None:
        got = np.asarray(got, np.float64)
        ref = np.asarray(ref, np.float64)
        err = np.abs(got - ref)
        bound = TIGHT_ATOL_ABSW + TIGHT_U_ABSW * np.asarray(absw, np.float64)
        worst = np.unravel_index(np.argmax(err - bound), err.shape)
        assert np.all(err <= bound), (f"{what} (fused semantics, weighted-|v| bar): "
                                      f"|d|={err[worst]:.3e} > {bound[worst]:.3e} at "
                                      f"{tuple(int(i) for i in worst)} (ref {ref[worst]:.4f})")
        return float(err.max()), 0.0
    atol, rtol = (TIGHT_ATOL_MFMA, TIGHT_RTOL_MFMA) if mfma else (TIGHT_ATOL, TIGHT_RTOL)
    return assert_close(got, ref, atol, rtol, what=what + " (fused semantics)")
