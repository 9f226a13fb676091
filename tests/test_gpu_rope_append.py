"""GPU parity of the one-token fused append (cq_qkv_rope_append, through
ChronoQuantCache.fused_decode_append).

It replaces two steps whose own parity is tested elsewhere:

- cq_qkv_norm_rope (test_gpu_model_ops.py, against torch fp32);
- cq_append through update_and_fetch (the codec and append tests, against
  the oracle).

Bar: bit-identical queries, cache arrays (every written I-frame row, packed
P-frame row and scale) and length vector.  Steps cross I-frame boundaries of
both strides (new I-frames and P-frames against cached anchors).  They run
with host offsets, and with device positions that differ per sequence (one
sequence rewriting earlier positions).  The codec settings are
Full-Throttle-like (4/3 bits, a V dead zone).
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rope_tables(max_pos, theta=1e6, D=128):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None]
    return ang.cos().float().cuda(), ang.sin().float().cuda()


def _bits(t):
    return t.view({1: torch.int8, 2: torch.int16, 4: torch.int32}[t.element_size()])


def _written(cache, b, T):
    """Sequence b's rows of every array holding positions [0, T)."""
    from chronoquant_mlx_amd.cache import _num_keyframes, _num_pframes
    out = []
    for comp in ("k", "v"):
        s = cache._stride(comp)
        nk, npf = _num_keyframes(T, s), _num_pframes(T, s)
        out += [cache._kf[comp][b, :, :nk], cache._pk[comp][b, :, :npf],
                cache._sc[comp][b, :, :npf]]
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("device_pos", [False, True])
@pytest.mark.parametrize("dense", [False, True])  # the 3-bit V rows stored dense
def test_fused_append_matches_two_steps(dtype, device_pos, dense):
    from chronoquant_mlx_amd import ChronoQuantCache
    from chronoquant_mlx_amd.models import fused
    B, H, G, D, T0, steps = 3, 2, 4, 128, 13, 19
    nq = G * H
    g = torch.Generator(device="cuda").manual_seed(7 + int(device_pos))
    cos, sin = _rope_tables(256)
    qw = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).to(dtype)
    ref, fus = [ChronoQuantCache(stride_k=4, stride_v=8, delta_bits_k=4, delta_bits_v=3,
                                 dead_zone_k=0.0, dead_zone_v=0.05, dense_residuals=dense)
                for _ in range(2)]
    k0 = torch.randn(B, H, T0, D, device="cuda", generator=g).to(dtype)
    v0 = torch.randn(B, H, T0, D, device="cuda", generator=g).to(dtype)
    for c in (ref, fus):
        c.update_and_fetch(k0, v0)
    if device_pos:
        # sequence 1 and 2 rewrite earlier positions (their anchors exist)
        pos = torch.tensor([T0, T0 - 4, T0 - 9], dtype=torch.int32, device="cuda")
        lens_r = torch.full((B,), -1, dtype=torch.int32, device="cuda")
        lens_f = torch.full((B,), -1, dtype=torch.int32, device="cuda")
        ref.bind_device_position(pos, T0 + steps + 8, lengths=lens_r)
        fus.bind_device_position(pos, T0 + steps + 8, lengths=lens_f)
    top = [T0] * B  # positions [0, top[b]) of sequence b are written
    for step in range(steps):
        qkv = (2 * torch.randn(B, 1, (nq + 2 * H) * D, device="cuda", generator=g)).to(dtype)
        if device_pos:
            positions = pos.long()[:, None]
        else:
            positions = torch.tensor([ref.offset], device="cuda")
        q_r, k_r, v_r = fused.qkv_norm_rope(qkv, nq, H, qw, kw, cos, sin, positions, 1e-6)
        ref.update_and_fetch(k_r, v_r)
        q_f = fus.fused_decode_append(qkv, nq, qw, kw, cos, sin, positions, 1e-6)
        assert q_f is not None and q_f.shape == q_r.shape == (B, nq, 1, D)
        assert torch.equal(_bits(q_f), _bits(q_r)), f"step {step}: q"
        if device_pos:
            assert torch.equal(lens_f, lens_r) and torch.equal(lens_f, pos + 1), f"step {step}"
            top = [max(top[b], int(pos[b]) + 1) for b in range(B)]
            pos += 1
            ref.advance(1)
            fus.advance(1)
        else:
            assert fus.offset == ref.offset
            top = [ref.offset] * B
        for b in range(B):
            for x, y in zip(_written(ref, b, top[b]), _written(fus, b, top[b])):
                assert torch.equal(_bits(x), _bits(y)), f"step {step}: sequence {b}"


def test_fused_append_declines_unsupported_shapes():
    # head_dim 64, or a batch the cache was not shaped for: None (the model
    # then runs the two steps)
    from chronoquant_mlx_amd import ChronoQuantCache
    cos, sin = _rope_tables(64, D=64)
    c = ChronoQuantCache()
    q = torch.zeros(1, 1, 64 * 4, dtype=torch.float16, device="cuda")
    pos = torch.tensor([0], device="cuda")
    assert c.fused_decode_append(q, 2, None, None, cos, sin, pos, 1e-6) is None  # not shaped
    k = torch.randn(1, 1, 5, 64, dtype=torch.float16, device="cuda")
    c.update_and_fetch(k, k)
    assert c.fused_decode_append(q, 2, None, None, cos, sin, pos, 1e-6) is None  # D = 64
    cos, sin = _rope_tables(64)
    c = ChronoQuantCache()
    k = torch.randn(2, 1, 5, 128, dtype=torch.float16, device="cuda")
    c.update_and_fetch(k, k)
    q = torch.zeros(1, 1, 128 * 4, dtype=torch.float16, device="cuda")
    assert c.fused_decode_append(q, 2, None, None, cos, sin, pos, 1e-6) is None  # B = 1 vs 2
    assert c.offset == 5 and not math.isnan(float(c._kf["k"][0, 0, 0, 0]))
