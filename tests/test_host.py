"""Host-side logic that needs no GPU: counting, masks, factories, patch routing."""
import sys
import types

import pytest
import torch

import chronoquant_mlx_amd as cq
from chronoquant_mlx_amd import cache as cache_mod
from chronoquant_mlx_amd import host, patch


def test_counts_match_reference_formulas():
    C = cq.ChronoQuantCache
    assert C._num_keyframes(0, 32) == 0 and C._num_pframes(0, 32) == 0
    assert C._num_keyframes(1, 32) == 1 and C._num_pframes(1, 32) == 0
    assert C._num_keyframes(33, 32) == 2 and C._num_pframes(33, 32) == 31
    assert C._num_keyframes(16384, 32) == 512 and C._num_pframes(16384, 8) == 14336


def test_make_causal_mask():
    assert cache_mod.make_causal_mask(10, 1) is None
    assert cache_mod.make_causal_mask(10, 4) == "causal"
    m = cache_mod.make_causal_mask(10, 4, return_array=True)
    assert m.shape == (4, 10) and m[0, 6] and not m[0, 7] and m[3].all()


def test_full_throttle_config():
    assert cq.FULL_THROTTLE_V3_CONFIG == {"stride_k": 64, "stride_v": 32, "delta_bits_k": 4,
                                          "delta_bits_v": 3, "dead_zone_k": 0.0,
                                          "dead_zone_v": 0.05}


class _Model:
    layers = [object()] * 5


def test_factories_and_per_layer_bits():
    caches = cq.create_chronoquant_caches(_Model(), per_layer_v_bits=[4, 3, 2])
    assert len(caches) == 5 and all(isinstance(c, cq.ChronoQuantCache) for c in caches)
    assert [c.layer_idx for c in caches] == list(range(5))
    assert [c.delta_bits_v for c in caches] == [4, 3, 2, 4, 4]
    # the lazy V codec reads per_layer_v_bits[min(layer_idx, len-1)] (cache.py:192-196)
    assert [c._get_codec_for_v().delta_bits for c in caches] == [4, 3, 2, 2, 2]
    ft = cq.create_full_throttle_caches(_Model())
    assert ft[0].stride_k == 64 and ft[0].stride_v == 32 and ft[0]._get_codec_for_v().delta_bits == 3
    assert ft[0].dead_zone_v == 0.05 and ft[0].use_fused


def test_defaults_match_reference():
    c = cq.ChronoQuantCache()
    assert (c.stride_k, c.stride_v, c.delta_bits_k, c.delta_bits_v) == (32, 8, 4, 4)
    assert (c.dead_zone_k, c.dead_zone_v, c.use_fused) == (0.0, 0.05, True)
    assert c.offset == 0 and c.empty() and c.state == [] and c.nbytes == 0
    assert not c.is_trimmable() and c.meta_state == ""


def test_codec_rejects_unsupported_bits():
    from chronoquant_mlx_amd.codec import ChronoQuantCodec
    with pytest.raises(ValueError):
        ChronoQuantCodec(delta_bits=5)


def test_patch_rebinds_registered_modules_and_reverts():
    mod = types.ModuleType("chronoquant_mlx_amd.models.fake_llm")
    mod.scaled_dot_product_attention = host.scaled_dot_product_attention
    sys.modules[mod.__name__] = mod
    try:
        cq.apply()
        cq.apply()  # idempotent
        assert host.scaled_dot_product_attention is patch._patched_sdpa
        assert mod.scaled_dot_product_attention is patch._patched_sdpa
        # non-ChronoQuant caches go to the original SDPA
        q = torch.randn(1, 2, 1, 8)
        k = torch.randn(1, 1, 3, 8)
        out = host.scaled_dot_product_attention(q, k, k, host.KVCache(), 0.3, None)
        ref = patch._original_sdpa(q, k, k, None, 0.3, None)
        assert torch.equal(out, ref)
        cq.revert()
        assert host.scaled_dot_product_attention is patch._original_sdpa
        assert mod.scaled_dot_product_attention is patch._original_sdpa
    finally:
        del sys.modules[mod.__name__]
        cq.revert()


def test_cpu_tensors_are_rejected():
    c = cq.ChronoQuantCache()
    k = torch.zeros(1, 2, 3, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        c.update_and_fetch(k, k)


def test_host_kvcache_protocol():
    c = host.KVCache()
    k = torch.randn(1, 2, 5, 4)
    a, b = c.update_and_fetch(k, k)
    assert c.offset == 5 and a.shape == (1, 2, 5, 4)
    a, b = c.update_and_fetch(k[:, :, :1], k[:, :, :1])
    assert c.offset == 6 and torch.equal(a[:, :, 5], k[:, :, 0])
    assert c.make_mask(1) is None and c.make_mask(3) == "causal"
