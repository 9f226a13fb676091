"""The HIP path against the committed golden vectors (tests/golden).

Append: keyframes, packed words and scales bit-exact, appended in one call
and token by token (decode-style streaming).  Decode: the fallback output
within the north-star bar (2e-3 + 1e-2|ref|) and the fused-kernel output
within the tight bar of the kernel that runs (MFMA for head_dim 128 and
strides >= 4, the portable kernel otherwise).
"""
import os

import numpy as np
import pytest
import torch

from tests.cqtest import assert_close, assert_tight, build_gpu_cache, to_gpu

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
ATTN = ["c0_small", "ft_v3_gqa", "bits3_dz02", "d72", "stride1"]


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def params(g, name):
    H, nq, T, D, sk, sv, bk, bv = (int(x) for x in g[f"{name}/params"])
    dzk, dzv = (float(x) for x in g[f"{name}/dead_zone"])
    return (H, nq, T, D), dict(stride_k=sk, stride_v=sv, bits_k=bk, bits_v=bv, dz_k=dzk, dz_v=dzv)


def check_state(cache, g, name):
    st = cache.state
    names = [("keyframes_k", 0), ("keyframes_v", 1), ("packed_k", 2), ("scales_k", 3),
             ("packed_v", 4), ("scales_v", 5)]
    for key, i in names:
        got = st[i][0].cpu().numpy()
        ref = g[f"{name}/{key}"]
        if got.dtype == np.float16:
            got, ref = got.view(np.uint16), ref.view(np.uint16)
        assert got.shape == ref.shape, (key, got.shape, ref.shape)
        assert np.array_equal(got, ref), f"{name}: {key} differs"


@pytest.mark.parametrize("name", ATTN)
def test_append_bulk(g, name):
    (H, nq, T, D), p = params(g, name)
    cache = build_gpu_cache(g[f"{name}/k"][None], g[f"{name}/v"][None], **p)
    check_state(cache, g, name)


@pytest.mark.parametrize("name", ["c0_small", "ft_v3_gqa", "stride1"])
def test_append_streaming(g, name):
    (H, nq, T, D), p = params(g, name)
    chunks = [1] * 10 + [T - 10]
    cache = build_gpu_cache(g[f"{name}/k"][None], g[f"{name}/v"][None], chunks=chunks, **p)
    check_state(cache, g, name)


@pytest.mark.parametrize("name", ATTN)
def test_decode(g, name):
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    (H, nq, T, D), p = params(g, name)
    cache = build_gpu_cache(g[f"{name}/k"][None], g[f"{name}/v"][None], **p)
    q = to_gpu(g[f"{name}/q"][None])
    out = chronoquant_sdpa_cache_kernel(q, cache, D ** -0.5).float().cpu().numpy()[0]
    assert_close(out, g[f"{name}/out_fallback"].astype(np.float64), what=name)
    mfma = D == 128 and min(p["stride_k"], p["stride_v"]) >= 4  # the MFMA kernel's domain
    assert_tight(out, g[f"{name}/out_fused"], what=name, mfma=mfma)
