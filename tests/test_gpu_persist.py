"""State save/load (the reference's state list, cache.py:220-255, written as
one safetensors file the way mlx_lm's save_prompt_cache lays it out)."""
import numpy as np
import pytest
import torch

from tests.cqtest import build_gpu_cache, to_gpu

pytestmark = pytest.mark.gpu


def _kv(seed, B, H, T, D):
    rng = np.random.default_rng(seed)
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    return k, v


def _same_state(a, b):
    sa, sb = a.state, b.state
    assert len(sa) == len(sb)
    for x, y in zip(sa, sb):
        assert x.shape == y.shape and x.dtype == y.dtype
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.float16 else x,
                           y.view(torch.int16) if y.dtype == torch.float16 else y)
    assert a.offset == b.offset and a.nbytes == b.nbytes


@pytest.mark.parametrize("params", [dict(stride_k=32, stride_v=8),
                                    dict(stride_k=64, stride_v=32, bits_v=3, dz_v=0.05),
                                    dict(stride_k=1, stride_v=8)])
def test_round_trip_then_continue(tmp_path, params):
    from chronoquant_mlx_amd import load_prompt_cache, save_prompt_cache
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    B, H, T, D = 2, 4, 400, 128
    k, v = _kv(3, B, H, T + 100, D)
    a = build_gpu_cache(k[:, :, :T], v[:, :, :T], **params)
    f = str(tmp_path / "cache.safetensors")
    save_prompt_cache(f, [a], {"model": "test"})
    (b,), meta = load_prompt_cache(f, return_metadata=True)
    assert meta == {"model": "test"}
    assert (b.stride_k, b.stride_v, b.delta_bits_v, b.dead_zone_v) == \
        (a.stride_k, a.stride_v, a.delta_bits_v, a.dead_zone_v)
    _same_state(a, b)
    q = to_gpu(np.random.default_rng(4).standard_normal((B, 4 * H, D)).astype(np.float16))
    oa = chronoquant_sdpa_cache_kernel(q, a, D ** -0.5)
    ob = chronoquant_sdpa_cache_kernel(q, b, D ** -0.5)
    assert torch.equal(oa, ob)
    # appending to the reloaded cache continues exactly where the saved one was
    kn, vn = to_gpu(k[:, :, T:]), to_gpu(v[:, :, T:])
    a.update_and_fetch(kn, vn)
    b.update_and_fetch(kn, vn)
    _same_state(a, b)


def test_reference_four_tensor_list_with_stride_k_1():
    # the reference omits the keys' empty packed/scales pair when stride_k == 1
    from chronoquant_mlx_amd import ChronoQuantCache
    B, H, T, D = 1, 2, 70, 128
    k, v = _kv(5, B, H, T, D)
    a = build_gpu_cache(k, v, stride_k=1, stride_v=8)
    kf_k, kf_v, pk_k, sc_k, pk_v, sc_v = a.state
    assert pk_k.shape[2] == 0
    b = ChronoQuantCache(stride_k=1, stride_v=8)
    b.state = [kf_k, kf_v, pk_v, sc_v]
    _same_state(a, b)


def test_mixed_cache_kinds(tmp_path):
    from chronoquant_mlx_amd import load_prompt_cache, save_prompt_cache
    from chronoquant_mlx_amd.host import KVCache
    B, H, T, D = 1, 2, 50, 128
    k, v = _kv(6, B, H, T, D)
    a = build_gpu_cache(k, v, stride_k=32, stride_v=8)
    p = KVCache()
    p.update_and_fetch(to_gpu(k), to_gpu(v))
    f = str(tmp_path / "mixed.safetensors")
    save_prompt_cache(f, [a, p])
    a2, p2 = load_prompt_cache(f)
    _same_state(a, a2)
    assert isinstance(p2, KVCache) and p2.offset == T
    assert torch.equal(p2.state[0].cpu(), p.state[0].cpu())


@pytest.mark.parametrize("params", [dict(stride_k=64, stride_v=32, bits_v=3, dz_v=0.05),
                                    dict(stride_k=16, stride_v=8, bits_k=2, bits_v=3),
                                    dict(stride_k=32, stride_v=8)])
def test_dense_file_reloads_the_same_cache(tmp_path, params):
    # dense=True stores 2-/3-bit residual codes at their width; the reloaded
    # cache has the INT4-lane layout again, bit-identical, and attends alike
    import os

    from chronoquant_mlx_amd import load_prompt_cache, save_prompt_cache
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    B, H, T, D = 2, 4, 400, 128
    k, v = _kv(8, B, H, T, D)
    a = build_gpu_cache(k, v, **params)
    f_int4, f_dense = str(tmp_path / "int4.safetensors"), str(tmp_path / "dense.safetensors")
    save_prompt_cache(f_int4, [a])
    save_prompt_cache(f_dense, [a], dense=True)
    b = load_prompt_cache(f_dense)[0]
    _same_state(a, b)
    n_pf = {c: int(a.state[i].shape[2]) * B * H for c, i in (("k", 2), ("v", 4))}
    bits = {"k": params.get("bits_k", 4), "v": params.get("bits_v", 4)}
    saved = sum(n_pf[c] * (64 - D * bits[c] // 8) for c in "kv" if bits[c] < 4)
    assert os.path.getsize(f_int4) - os.path.getsize(f_dense) - saved in range(-256, 256)
    q = to_gpu(np.random.default_rng(9).standard_normal((B, 4 * H, D)).astype(np.float16))
    assert torch.equal(chronoquant_sdpa_cache_kernel(q, a, D ** -0.5), chronoquant_sdpa_cache_kernel(q, b, D ** -0.5))
