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


def test_array_mask_fallback():
    # attention.py:18-19: a boolean mask keeps scores where True and puts
    # finfo(fp16).min elsewhere.  Pinned by: the causal boolean mask equals the
    # "causal" string; an all-True mask changes nothing; a window of at least
    # T equals causal; a mask keeping one key per query returns that key's
    # value row exactly; the C and numpy restatements agree bit for bit.
    from chronoquant_mlx_amd.cache import make_causal_mask
    rng = np.random.default_rng(5)
    nq, H, T, D, Tq = 4, 2, 40, 32, 6
    q = rng.standard_normal((nq, Tq, D)).astype(np.float16)
    k = rng.standard_normal((H, T, D)).astype(np.float16)
    v = rng.standard_normal((H, T, D)).astype(np.float16)
    u16 = lambda a: a.view(np.uint16)
    causal_arr = make_causal_mask(T, Tq, return_array=True).numpy()
    assert causal_arr.shape == (Tq, T)
    ref = O.sdpa_fallback(q, k, v, 0.3, causal=True)
    assert np.array_equal(u16(O.sdpa_fallback(q, k, v, 0.3, mask=causal_arr)), u16(ref))
    assert np.array_equal(u16(O.sdpa_fallback(q, k, v, 0.3, mask=np.ones((Tq, T), bool))),
                          u16(O.sdpa_fallback(q, k, v, 0.3)))
    wide = make_causal_mask(T, Tq, return_array=True, window_size=T).numpy()
    assert np.array_equal(wide, causal_arr)
    one = np.zeros((Tq, T), bool)
    pick = rng.integers(0, T, size=Tq)
    one[np.arange(Tq), pick] = True
    out = O.sdpa_fallback(q, k, v, 0.3, mask=one)
    for j in range(nq):
        assert np.array_equal(u16(out[j]), u16(v[j // (nq // H), pick]))
    win = make_causal_mask(T, Tq, window_size=4).numpy()
    assert win.shape == (Tq, T) and win.sum(axis=1).tolist() == [4] * Tq
    assert np.array_equal(u16(O.sdpa_fallback(q, k, v, 0.3, mask=win)),
                          u16(N.sdpa_fallback(q, k, v, 0.3, mask=win)))


def test_fused_weighted_abs_scale():
    # With stride 1 every token is an I-frame, so the fused-semantics oracle
    # is textbook attention over the fp16 keys/values with q' = fp16(q *
    # fp16(scale)); its absw output is the softmax-weighted mean of |v|.
    # Both against a float64 numpy restatement.
    rng = np.random.default_rng(1)
    H, D, T, nq = 2, 64, 300, 4
    k = np.cumsum(rng.standard_normal((H, T, D)) * 0.1, axis=1).astype(np.float16)
    v = np.cumsum(rng.standard_normal((H, T, D)) * 0.1, axis=1).astype(np.float16)
    ck = O.OracleComponent(H, D, 1, 4, 0.0, capacity=T)
    cv = O.OracleComponent(H, D, 1, 4, 0.0, capacity=T)
    ck.append(k)
    cv.append(v)
    q = rng.standard_normal((nq, D)).astype(np.float16)
    out, absw = O.sdpa_fused(q, ck, cv, 0.125, return_absw=True)
    kv = [j // (nq // H) for j in range(nq)]
    qs = (q.astype(np.float32) * np.float32(np.float16(0.125))).astype(np.float16)
    s = np.einsum("jd,jtd->jt", qs.astype(np.float64), k.astype(np.float64)[kv])
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ref = np.einsum("jt,jtd->jd", p, v.astype(np.float64)[kv])
    refa = np.einsum("jt,jtd->jd", p, np.abs(v.astype(np.float64))[kv])
    assert np.abs(out - ref).max() < 1e-6 and np.abs(absw - refa).max() < 1e-6
    assert np.all(absw >= np.abs(out) - 1e-6)


def test_bf16_query_fallback():
    # attention.py:61-74 with bf16 queries: q' = bf16(q * bf16(scale)), fp32
    # scores and weights, one rounding to bf16.  Pinned by: binary64
    # attention on the same q' (exact in fp16 here) rounded to bf16 agrees to
    # within one bf16 rounding; the causal mask equals truncation; a mask
    # keeping one key per query returns bf16(that value row) exactly.
    rng = np.random.default_rng(6)
    nq, H, T, D, Tq, scale = 4, 2, 50, 32, 3, 0.3
    qf = rng.standard_normal((nq, Tq, D)).astype(np.float32)
    qb = O.f32_to_bf16(qf)
    k = rng.standard_normal((H, T, D)).astype(np.float16)
    v = rng.standard_normal((H, T, D)).astype(np.float16)
    out = O.sdpa_fallback_bf16q(qb, k, v, scale)
    qprime = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(qb) * O.bf16_to_f32(O.f32_to_bf16(
        np.float32(scale)))))
    assert np.array_equal(qprime.astype(np.float16).astype(np.float32), qprime)
    got = O.bf16_to_f32(out).astype(np.float64)
    for i in range(Tq):
        ex = O.sdpa_exact(np.ascontiguousarray(qprime[:, i].astype(np.float16)), k, v, 1.0)
        assert np.all(np.abs(got[:, i] - ex) <= 2.0 ** -8 * np.abs(ex) + 1e-30), i
    causal = O.sdpa_fallback_bf16q(qb, k, v, scale, causal=True)
    for i in range(Tq):
        Ti = T - Tq + i + 1
        ref = O.sdpa_fallback_bf16q(np.ascontiguousarray(qb[:, i: i + 1]),
                                    np.ascontiguousarray(k[:, :Ti]),
                                    np.ascontiguousarray(v[:, :Ti]), scale)
        assert np.array_equal(causal[:, i], ref[:, 0])
    one = np.zeros((Tq, T), bool)
    pick = rng.integers(0, T, size=Tq)
    one[np.arange(Tq), pick] = True
    sel = O.sdpa_fallback_bf16q(qb, k, v, scale, mask=one)
    for j in range(nq):
        assert np.array_equal(sel[j], O.f32_to_bf16(v[j // (nq // H), pick].astype(np.float32)))


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
