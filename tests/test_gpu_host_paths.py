"""GPU checks of the host-side paths around the kernels: the kernel operand
accessors (cache.py:162-190), the array-mask and windowed reconstruct
fallback (cache.py:7-15 -> attention.py:18-20, 61-74), and the codec's
dequantize_delta (codec.py:67-73)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import assert_close, build_gpu_cache, build_oracle, to_gpu

pytestmark = pytest.mark.gpu


def _data(seed, H, T, D=128):
    rng = np.random.default_rng(seed)
    k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    return k, v


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("T,sk,sv", [(300, 32, 8), (1, 32, 8), (50, 1, 8), (40, 64, 1)])
def test_kernel_accessors(T, sk, sv):
    # squeezed active slices [H, ., .] (cache.py:162-168); a component with no
    # P-frame rows yet gives the zero placeholders [H, 1, 1] uint32 and
    # [H, 1] fp16 (cache.py:170-190: the reference's packed/scales stay None
    # until its first P-frame)
    H, D = 4, 128
    params = dict(stride_k=sk, stride_v=sv)
    k, v = _data(T + sk, H, T, D)
    cache = build_gpu_cache(k, v, **params)
    ck, cv = build_oracle(k[0], v[0], **params)
    for name, comp in (("k", ck), ("v", cv)):
        kf, pk, sc = comp.active()
        got_kf = getattr(cache, f"kernel_keyframes_{name}")()
        got_pk = getattr(cache, f"kernel_packed_{name}")()
        got_sc = getattr(cache, f"kernel_scales_{name}")()
        assert got_kf.shape == (H, kf.shape[1], D)
        assert np.array_equal(_u16(got_kf), kf.view(np.uint16))
        if pk.shape[1] == 0:
            assert got_pk.shape == (H, 1, 1) and got_pk.dtype == torch.uint32
            assert got_sc.shape == (H, 1) and got_sc.dtype == torch.float16
            assert not got_pk.cpu().numpy().any() and not got_sc.float().cpu().numpy().any()
        else:
            assert got_pk.shape == (H, pk.shape[1], D // 8) and got_sc.shape == (H, pk.shape[1])
            assert np.array_equal(got_pk.cpu().numpy(), pk)
            assert np.array_equal(_u16(got_sc), sc.view(np.uint16))


@pytest.mark.parametrize("window", [None, 16, 1000])
def test_array_mask_fallback(window):
    # make_mask with return_array (or a window shorter than the chunk) gives a
    # boolean array; chronoquant_sdpa then takes the reconstruct fallback
    # with where(mask, scores, finfo.min), checked against the oracle's
    # fallback with the same mask
    from chronoquant_mlx_amd import chronoquant_sdpa
    H, G, T, L, D = 2, 4, 300, 40, 128
    params = dict(stride_k=32, stride_v=8)
    k, v = _data(17, H, T, D)
    cache = build_gpu_cache(k, v, **params)
    mask = cache.make_mask(L, return_array=window is None, window_size=window)
    if window is not None and window >= L:
        assert mask == "causal"  # mlx_lm's rule: a window no shorter than the chunk
        mask = cache.make_mask(L, return_array=True, window_size=window)
    assert isinstance(mask, torch.Tensor) and mask.shape == (L, T)
    q = np.random.default_rng(18).standard_normal((1, G * H, L, D)).astype(np.float16)
    out = chronoquant_sdpa(to_gpu(q), None, None, cache, D ** -0.5, mask=mask)
    ck, cv = build_oracle(k[0], v[0], **params)
    ref = O.sdpa_fallback(q[0], ck.reconstruct(), cv.reconstruct(), D ** -0.5,
                          mask=mask.cpu().numpy())
    assert_close(out.float().cpu().numpy()[0], ref.astype(np.float64), what=f"window={window}")


def test_dequantize_delta():
    # fp16(code) * fp16 scale, one fp16 rounding (the product of two fp16
    # values is exact in fp32, so numpy's fp16 multiply is the reference)
    from chronoquant_mlx_amd.codec import ChronoQuantCodec
    rng = np.random.default_rng(4)
    codes = rng.integers(-8, 8, size=(2, 3, 5, 128)).astype(np.int8)
    scales = (rng.lognormal(-4, 2, size=(2, 3, 5, 1))).astype(np.float16)
    scales[0, 0, 0, 0] = np.float16(6e-8)  # subnormal scale
    got = ChronoQuantCodec().dequantize_delta(torch.from_numpy(codes).cuda(),
                                              torch.from_numpy(scales).cuda())
    ref = codes.astype(np.float16) * scales
    assert got.dtype == torch.float16
    assert np.array_equal(_u16(got), ref.view(np.uint16))


def test_bound_cache_takes_only_the_fused_decode():
    # A cache bound to device positions (graph-captured decode loops) has a
    # host offset that trails the device one.  chronoquant_sdpa must serve it
    # with the fused decode over the device lengths, also when the host
    # offset is still 0, and refuse the paths that read the host offset.
    from chronoquant_mlx_amd import ChronoQuantCache, chronoquant_sdpa
    H, G, D = 2, 4, 128
    cache = ChronoQuantCache(stride_k=32, stride_v=8, dead_zone_v=0.0)
    empty = torch.zeros(1, H, 0, D, dtype=torch.float16, device="cuda")
    cache.update_and_fetch(empty, empty)  # shapes the cache, appends nothing
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    cache.bind_device_position(pos, max_len=64)
    rng = np.random.default_rng(30)
    k, v = _data(31, H, 2, D)
    q = to_gpu(rng.standard_normal((1, G * H, 1, D)))
    cache.update_and_fetch(to_gpu(k[:, :, :1]), to_gpu(v[:, :, :1]))
    assert cache.offset == 0
    out = chronoquant_sdpa(q, None, None, cache, D ** -0.5)
    # one cached token: attention returns its value row (an I-frame: exact)
    want = np.repeat(v[0, :, 0], G, axis=0)
    assert np.array_equal(_u16(out[0, :, 0].contiguous()), want.view(np.uint16))
    with pytest.raises(ValueError):
        chronoquant_sdpa(q.expand(1, G * H, 3, D).contiguous(), None, None, cache, D ** -0.5,
                         mask="causal")
    cache.bind_device_position(None)


@pytest.mark.parametrize("prefill", [False, True])
def test_torch_graph_recipe(prefill):
    # torch's recipe: warm up on a side stream, capture with
    # torch.cuda.graph(g) (torch's own capture stream, whose split workspace
    # is then allocated under capture); replays with other library calls
    # between them must each equal the eager result
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel, chronoquant_sdpa_cache_kernel
    H, G, T, D = 8, 4, 3000, 128
    k, v = _data(40 + prefill, H, T, D)
    cache = build_gpu_cache(k, v, stride_k=32, stride_v=8)
    rng = np.random.default_rng(41)
    if prefill:
        q = to_gpu(rng.standard_normal((1, G * H, 256, D)))
        run = lambda: chronoquant_prefill_kernel(q, cache, D ** -0.5, causal=True)
    else:
        q = to_gpu(rng.standard_normal((1, G * H, D)))
        run = lambda: chronoquant_sdpa_cache_kernel(q, cache, D ** -0.5)
    ref = run().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = run()
    k2, v2 = _data(42, 2, 700, D)
    other = build_gpu_cache(k2, v2, stride_k=16, stride_v=4)
    q2 = to_gpu(rng.standard_normal((1, 8, D)))
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        chronoquant_sdpa_cache_kernel(q2, other, D ** -0.5)  # eager work between the replays
