"""Pins the oracle's attention (reference attention.py:8-74, MSL kernels.py:79-228).

The fallback restatement keeps the reference's fp16 rounding points; it is
checked against binary64 textbook attention (tolerance = the decode parity
bar, max-abs 2e-3 / rel 1e-2) and against closed-form special cases.
"""
import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O

ATOL, RTOL = 2e-3, 1e-2


def close(a, b, atol=ATOL, rtol=RTOL):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    err = np.abs(a - b)
    assert err.max() <= atol, err.max()
    assert np.linalg.norm(a - b) <= rtol * np.linalg.norm(b) + 1e-12


def test_single_token_returns_v0():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((4, 1, 64)).astype(np.float16)
    k = rng.standard_normal((2, 1, 64)).astype(np.float16)
    v = rng.standard_normal((2, 1, 64)).astype(np.float16)
    out = O.sdpa_fallback(q, k, v, 0.125)
    assert np.array_equal(out[:, 0].view(np.uint16), np.repeat(v[:, 0], 2, axis=0).view(np.uint16))


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(1)
    T = 64
    q = rng.standard_normal((2, 1, 32)).astype(np.float16)
    k = np.repeat(rng.standard_normal((1, 1, 32)), T, axis=1).astype(np.float16)
    v = rng.standard_normal((1, T, 32)).astype(np.float16)
    out = O.sdpa_fallback(q, k, v, 0.2)
    mean = v.astype(np.float64).mean(axis=1)
    # weights are fp16(1/64) = exact: output is the exact mean rounded to fp16
    assert np.allclose(out[:, 0].astype(np.float64), mean, atol=1e-3)


def test_dominant_score_selects_row():
    D, T = 16, 10
    q = np.zeros((1, 1, D), np.float16)
    q[0, 0, 0] = 8.0
    k = np.zeros((1, T, D), np.float16)
    k[0, 3, 0] = 8.0           # score 64*scale(=1) vs 0 elsewhere
    v = np.arange(T * D, dtype=np.float32).reshape(1, T, D).astype(np.float16) / 64
    out = O.sdpa_fallback(q, k, v, 1.0)
    assert np.array_equal(out[0, 0].view(np.uint16), v[0, 3].view(np.uint16))


def test_gqa_mapping():
    # q head j reads kv head j // (nq/H): permuting kv heads permutes outputs
    rng = np.random.default_rng(2)
    nq, H, T, D = 8, 2, 40, 32
    q = rng.standard_normal((nq, 1, D)).astype(np.float16)
    k = rng.standard_normal((H, T, D)).astype(np.float16)
    v = rng.standard_normal((H, T, D)).astype(np.float16)
    a = O.sdpa_fallback(q, k, v, 0.17)
    b = O.sdpa_fallback(np.concatenate([q[4:], q[:4]]), k[::-1].copy(), v[::-1].copy(), 0.17)
    assert np.array_equal(a.view(np.uint16), np.concatenate([b[4:], b[:4]]).view(np.uint16))


def test_causal_mask_equals_truncation():
    rng = np.random.default_rng(3)
    nq, H, T, D, Tq = 4, 2, 30, 32, 5
    q = rng.standard_normal((nq, Tq, D)).astype(np.float16)
    k = rng.standard_normal((H, T, D)).astype(np.float16)
    v = rng.standard_normal((H, T, D)).astype(np.float16)
    out = O.sdpa_fallback(q, k, v, 0.2, causal=True)
    for i in range(Tq):
        Ti = T - Tq + i + 1
        ref = O.sdpa_fallback(np.ascontiguousarray(q[:, i: i + 1]),
                              np.ascontiguousarray(k[:, :Ti]), np.ascontiguousarray(v[:, :Ti]), 0.2)
        assert np.array_equal(out[:, i].view(np.uint16), ref[:, 0].view(np.uint16))
    assert np.array_equal(out.view(np.uint16),
                          N.sdpa_fallback(q, k, v, 0.2, causal=True).view(np.uint16))


@pytest.mark.parametrize("T", [1, 7, 300, 4096])
def test_fallback_and_fused_within_bar_of_exact(T):
    from chronoquant_mlx_amd import synth
    cfg = synth.CONFIGS["c0"]
    k, v = synth.make_kv(cfg, T=T)
    q = synth.make_q(cfg)[0]
    H, D = cfg.n_kv_heads, cfg.head_dim
    ck = O.OracleComponent(H, D, cfg.stride_k, 4, 0.0, capacity=T)
    cv = O.OracleComponent(H, D, cfg.stride_v, 4, 0.0, capacity=T)
    ck.append(k[0])
    cv.append(v[0])
    scale = D ** -0.5
    rk, rv = ck.reconstruct(), cv.reconstruct()
    exact = O.sdpa_exact(q, rk, rv, scale)
    fb = O.sdpa_fallback(q[:, None], rk, rv, scale)[:, 0]
    fused = O.sdpa_fused(q, ck, cv, scale)
    close(fb, exact)
    close(fused, exact)
    # the compressed cache stays close to attention over the raw fp16 stream
    raw = O.sdpa_exact(q, k[0], v[0], scale)
    assert np.linalg.norm(exact - raw) < 0.05 * np.linalg.norm(raw)
