"""GPU parity of the chunked-prefill kernel (cq_prefill_attn) against the
oracle's restatement of the reference's reconstruct fallback for q_len > 1
(attention.py:61-74 with the causal mask of attention.py:12-16, over
cache.py:131-160), and against the torch fallback path of chronoquant_sdpa.

Bar: |got - ref| <= 2e-3 + 1e-2 |ref| elementwise and relative L2 <= 1e-2
(the north-star attention tolerance).  The kernel rounds scores to fp16 as
the fallback does; its softmax is the online form with fp16 weights.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import assert_close, build_gpu_cache, build_oracle, to_gpu

pytestmark = pytest.mark.gpu


def _data(seed, B, H, T, D):
    rng = np.random.default_rng(seed)
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    return k, v


def _check(B, H, G, T, L, params, causal=True, seed=0, chunks=None):
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel
    D = 128
    k, v = _data(seed, B, H, T, D)
    q = np.random.default_rng(seed + 1).standard_normal((B, G * H, L, D)).astype(np.float16)
    cache = build_gpu_cache(k, v, chunks=chunks, **params)
    scale = D ** -0.5
    out = chronoquant_prefill_kernel(to_gpu(q), cache, scale, causal=causal).float().cpu().numpy()
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        ref = O.sdpa_fallback(q[b], ck.reconstruct(), cv.reconstruct(), scale, causal=causal)
        assert_close(out[b], ref.astype(np.float64), what=f"b={b} T={T} L={L} {params}")
    return out


@pytest.mark.parametrize("G,H", [(1, 8), (4, 8), (8, 2), (16, 1)])
def test_gqa_ratios(G, H):
    _check(1, H, G, 700, 128, dict(stride_k=32, stride_v=8), seed=G)


@pytest.mark.parametrize("params", [dict(stride_k=64, stride_v=32, bits_v=3, dz_v=0.05),
                                    dict(stride_k=1, stride_v=8),
                                    dict(stride_k=5, stride_v=12),
                                    dict(stride_k=4, stride_v=4, bits_k=3, bits_v=3, dz_k=0.2,
                                         dz_v=0.2),
                                    # power-of-two strides above 64 (offsets recomputed per
                                    # block, not stepped) and at 64 on both components
                                    dict(stride_k=128, stride_v=256),
                                    dict(stride_k=64, stride_v=64)])
def test_codec_settings(params):
    _check(1, 2, 4, 600, 100, params, seed=7)


@pytest.mark.parametrize("T,L", [(2, 2), (65, 64), (64, 64), (513, 512), (1000, 37), (300, 300)])
def test_lengths(T, L):
    # chunks that do not fill a position block, whole prompts, block edges
    _check(1, 2, 4, T, L, dict(stride_k=32, stride_v=8), seed=T + L)


def test_batch_and_full_attention():
    _check(2, 2, 4, 500, 96, dict(stride_k=32, stride_v=8), causal=False, seed=3)
    _check(2, 2, 4, 500, 96, dict(stride_k=32, stride_v=8), causal=True, seed=4)


def test_chunked_prefill_sequence():
    # the prompt arrives in 3 chunks; after each append the chunk's queries
    # attend causally to everything cached so far
    from chronoquant_mlx_amd import ChronoQuantCache
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel
    H, G, D, T = 2, 4, 128, 640
    params = dict(stride_k=32, stride_v=8)
    k, v = _data(9, 1, H, T, D)
    q = np.random.default_rng(10).standard_normal((1, G * H, T, D)).astype(np.float16)
    cache = ChronoQuantCache(stride_k=32, stride_v=8, dead_zone_v=0.0)
    ck, cv = build_oracle(k[0], v[0], **params)
    rk, rv = ck.reconstruct(), cv.reconstruct()
    pos = 0
    for L in (200, 256, 184):
        cache.update_and_fetch(to_gpu(k[:, :, pos:pos + L]), to_gpu(v[:, :, pos:pos + L]))
        out = chronoquant_prefill_kernel(to_gpu(q[:, :, pos:pos + L]), cache, D ** -0.5)
        ref = O.sdpa_fallback(q[0, :, pos:pos + L], rk[:, :pos + L], rv[:, :pos + L], D ** -0.5,
                              causal=True)
        assert_close(out.float().cpu().numpy()[0], ref.astype(np.float64), what=f"chunk at {pos}")
        pos += L


@pytest.mark.parametrize("mask", ["causal", None])
def test_sdpa_routes_prefill_and_matches_fallback(mask):
    from chronoquant_mlx_amd import attention as A
    H, G, T, L, D = 2, 4, 400, 64, 128
    params = dict(stride_k=32, stride_v=8)
    k, v = _data(11, 1, H, T, D)
    cache = build_gpu_cache(k, v, **params)
    q = to_gpu(np.random.default_rng(12).standard_normal((1, G * H, L, D)).astype(np.float16))
    A.PREFILL_KERNEL = True
    try:
        got = A.chronoquant_sdpa(q, None, None, cache, D ** -0.5, mask=mask)
        A.PREFILL_KERNEL = False
        ref = A.chronoquant_sdpa(q, None, None, cache, D ** -0.5, mask=mask)
    finally:
        A.PREFILL_KERNEL = True
    assert_close(got.float().cpu().numpy(), ref.float().cpu().numpy().astype(np.float64),
                 what=f"mask={mask}")


@pytest.mark.parametrize("params", [dict(stride_k=64, stride_v=32, bits_v=3, dz_v=0.05),
                                    dict(stride_k=5, stride_v=12)])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_queries(causal, params):
    # bf16 queries: q' = bf16(q * bf16(scale)), fp32 scores (the reference's
    # bf16 x fp16 promotion), bf16 output; against the oracle's bf16-query
    # fallback and, as a second reading, the fp16 fallback on the same q'
    # (exact in fp16) with scale 1.  Strides 5 / 12 take the float-reciprocal
    # token -> anchor path.
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel
    B, H, G, T, L, D = 1, 2, 4, 700, 130, 128
    k, v = _data(21, B, H, T, D)
    q32 = np.random.default_rng(22).standard_normal((B, G * H, L, D)).astype(np.float32)
    cache = build_gpu_cache(k, v, **params)
    qb = torch.from_numpy(q32).to("cuda").to(torch.bfloat16)
    out = chronoquant_prefill_kernel(qb, cache, D ** -0.5, causal=causal)
    assert out.dtype == torch.bfloat16
    qprime = (qb.cpu() * torch.tensor(D ** -0.5, dtype=torch.bfloat16)).to(torch.float16).numpy()
    ck, cv = build_oracle(k[0], v[0], **params)
    rk, rv = ck.reconstruct(), cv.reconstruct()
    ref = O.sdpa_fallback(qprime[0], rk, rv, 1.0, causal=causal)
    got = out.float().cpu().numpy()[0]
    assert_close(got, ref.astype(np.float64), what=f"causal={causal}")
    qbits = qb.cpu().view(torch.int16).numpy().view(np.uint16)[0]
    ref32 = O.bf16_to_f32(O.sdpa_fallback_bf16q(qbits, rk, rv, D ** -0.5, causal=causal))
    assert_close(got, ref32.astype(np.float64), what=f"causal={causal} (bf16 fallback)")


@pytest.mark.parametrize("bf16", [False, True])
def test_split_keys_match_single_pass(bf16):
    # The kernel splits each query tile's key range over several workgroups
    # and merges their partials; without a workspace it runs one pass per
    # tile.  Both must agree (they differ only in where the online softmax
    # rounds its fp16 weights).
    from chronoquant_mlx_amd import _lib
    D, B, H, G, T, L = 128, 1, 8, 4, 3000, 512
    params = dict(stride_k=64, stride_v=32, bits_v=3, dz_v=0.05)
    k, v = _data(11, B, H, T, D)
    q = np.random.default_rng(12).standard_normal((B, G * H, L, D)).astype(np.float16)
    dt = torch.bfloat16 if bf16 else torch.float16
    cache = build_gpu_cache(k, v, dtype=torch.float16, **params)
    qt = to_gpu(q, dt).contiguous()
    lib = _lib.load()
    need = lib.cq_prefill_workspace_size(B, H, G * H, L, T)
    assert need > 0, "this shape should split its keys"
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = []
    for w in (ws, None):
        out = torch.empty_like(qt)
        for _ in range(2):  # the second call reuses the counters of the first
            _lib.call("cq_prefill_attn", cache._descriptor(), qt.data_ptr(), _lib.dtype_code(dt),
                      G * H, L, D ** -0.5, 1, T, out.data_ptr(),
                      None if w is None else w.data_ptr(), 0 if w is None else w.numel(),
                      _lib.stream_of(qt))
        outs.append(out.float().cpu().numpy())
    torch.cuda.synchronize()
    # (the oracle tests above run split plans too: their shapes leave the
    # grid far below one resident generation)
    tol = 8e-3 if bf16 else 2e-3
    err = np.abs(outs[0] - outs[1]) - tol * np.abs(outs[1])
    assert err.max() <= tol, err.max()
