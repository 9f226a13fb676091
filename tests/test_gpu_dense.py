"""Dense residual rows in HBM (opt-in dense_residuals / CQ_PACK_DENSE): 2- and
3-bit components keep their codes at their own width instead of the
reference's INT4 lanes (the variable-bit packing the reference names as
what its INT4 lanes are not, README.md:57, patch.py:94-98).

Bars:
- rows: bit-identical to persist.dense_pack of the oracle's INT4 words (the
  at-rest dense format, itself pinned against the oracle's INT4 packer on the
  CPU), zero-padded to whole words; I-frames and scales bit-identical to the
  oracle;
- reconstruction: bit-identical to the oracle's (cache.py:131-156);
- attention: the decode bars of the INT4 layout (tests/cqtest.py): within
  the fallback bar of the oracle's reconstruct fallback and the tight bar of
  its fused semantics.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import (assert_close, assert_close_fallback, assert_tight, build_oracle,
                          to_gpu)

pytestmark = pytest.mark.gpu


def dense_cache(k, v, *, stride_k, stride_v, bits_k=4, bits_v=4, dz_k=0.0, dz_v=0.0,
                chunks=None, dtype=torch.float16, dense=True):
    from chronoquant_mlx_amd import ChronoQuantCache
    cache = ChronoQuantCache(stride_k=stride_k, stride_v=stride_v, delta_bits_k=bits_k,
                             delta_bits_v=bits_v, dead_zone_k=dz_k, dead_zone_v=dz_v,
                             dense_residuals=dense)
    T = k.shape[2]
    kt, vt = to_gpu(k, dtype), to_gpu(v, dtype)
    pos = 0
    for S in (chunks or [T]):
        cache.update_and_fetch(kt[:, :, pos: pos + S], vt[:, :, pos: pos + S])
        pos += S
    assert pos == T
    return cache


def expected_rows(int4_words: np.ndarray, D: int, bits: int) -> np.ndarray:
    """dense_pack of INT4 words, padded to whole uint32 words (bytes)."""
    from chronoquant_mlx_amd.persist import dense_pack
    stream = dense_pack(torch.from_numpy(np.ascontiguousarray(int4_words)), D, bits).numpy()
    rw = (D * bits + 31) // 32
    out = np.zeros(stream.shape[:-1] + (4 * rw,), np.uint8)
    out[..., : stream.shape[-1]] = stream
    return out


def assert_rows_match_oracle(cache, b, ck, cv, bits):
    D = cache._shape[2]
    st = cache.state
    for i, comp, fb in ((0, ck, bits[0]), (1, cv, bits[1])):
        kf, pk, sc = comp.active()
        assert np.array_equal(st[i][b].cpu().numpy().view(np.uint16), kf.view(np.uint16)), \
            f"keyframes[{i}] b={b}"
        assert np.array_equal(st[3 + 2 * i][b].cpu().numpy().view(np.uint16),
                              sc.view(np.uint16)), f"scales[{i}] b={b}"
        got = st[2 + 2 * i][b].contiguous().cpu().numpy()
        if fb < 4 and cache.dense_residuals:
            want = expected_rows(pk, D, fb)
            assert got.shape[-1] == (D * fb + 31) // 32
            assert np.array_equal(got.view(np.uint8), want), f"dense rows[{i}] b={b}"
        else:
            assert np.array_equal(got, pk), f"INT4 rows[{i}] b={b}"


def test_c2_shape_dense_v_rows_and_attention():
    # B=8, T=32768, Full-Throttle V3 (K 4-bit INT4, V 3-bit dense
    # rows), the plan bench.py's c2_dense line times
    from chronoquant_mlx_amd import synth
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    cfg = synth.CONFIGS["c2"]
    k, v = synth.make_kv(cfg)
    q = synth.make_q(cfg)
    params = dict(stride_k=cfg.stride_k, stride_v=cfg.stride_v, bits_k=cfg.delta_bits_k,
                  bits_v=cfg.delta_bits_v, dz_k=cfg.dead_zone_k, dz_v=cfg.dead_zone_v)
    dense = dense_cache(k, v, **params)
    int4 = dense_cache(k, v, **params, dense=False)
    assert dense.nbytes < int4.nbytes
    B, H, T, D = k.shape
    npf_v = T - ((T - 1) // cfg.stride_v + 1)
    assert int4.nbytes - dense.nbytes == B * H * npf_v * (64 - 48)
    # every sequence's dense V rows are dense_pack of the INT4 rows (which
    # the INT4 tests pin to the oracle); sequences 0 and 7 directly against
    # the oracle
    from chronoquant_mlx_amd.persist import dense_pack
    st_d, st_i = dense.state, int4.state
    assert torch.equal(st_d[2], st_i[2]) and torch.equal(st_d[3], st_i[3])
    want = dense_pack(st_i[4], D, 3)
    assert torch.equal(st_d[4].contiguous().view(torch.uint8), want)
    scale = D ** -0.5
    out_d = chronoquant_sdpa_cache_kernel(to_gpu(q), dense, scale).float().cpu().numpy()
    out_i = chronoquant_sdpa_cache_kernel(to_gpu(q), int4, scale).float().cpu().numpy()
    for b in (0, 7):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_rows_match_oracle(dense, b, ck, cv, (4, 3))
        fb = O.sdpa_fallback(q[b][:, None], ck.reconstruct(), cv.reconstruct(), scale)[:, 0]
        exact = O.sdpa_exact(q[b], ck.reconstruct(), cv.reconstruct(), scale)
        assert_close_fallback(out_d[b], fb, exact, what=f"c2 dense b={b}")
        fused, absw = O.sdpa_fused(q[b], ck, cv, scale, return_absw=True)
        assert_tight(out_d[b], fused, what=f"c2 dense b={b}", absw=absw)
    # the two layouts decode every sequence to the same values within the
    # parity bar (c2's outlier channels need the |v|-weighted tight bar,
    # applied above against the oracle)
    assert_close(out_d, out_i, what="c2 dense vs INT4 lanes")


@pytest.mark.parametrize("bits,D,strides", [((4, 3), 128, (32, 8)), ((3, 3), 128, (16, 4)),
                                            ((2, 3), 128, (64, 32)), ((3, 2), 72, (8, 8)),
                                            ((2, 2), 12, (4, 4)), ((3, 3), 5, (3, 5))])
def test_dense_layouts_rows_reconstruct_decode(bits, D, strides):
    # every packing path (row4 append at D=128, the one-row append
    # elsewhere), the reconstruction, and the decode routing (GQA-4 MFMA
    # instance for 4/3-bit at D=128, the portable kernel otherwise)
    rng = np.random.default_rng(sum(bits) * 100 + D)
    B, H, G, T = 2, 2, 4, 900
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=strides[0], stride_v=strides[1], bits_k=bits[0], bits_v=bits[1],
                  dz_v=0.05)
    cache = dense_cache(k, v, **params, chunks=[300, 1, 599])
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    out = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, D ** -0.5).float().cpu().numpy()
    rk, rv = cache.reconstruct_history()
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_rows_match_oracle(cache, b, ck, cv, bits)
        assert np.array_equal(rk[b].cpu().numpy().view(np.uint16),
                              ck.reconstruct().view(np.uint16)), f"reconstruct K b={b}"
        assert np.array_equal(rv[b].cpu().numpy().view(np.uint16),
                              cv.reconstruct().view(np.uint16)), f"reconstruct V b={b}"
        fb = O.sdpa_fallback(q[b][:, None], ck.reconstruct(), cv.reconstruct(), D ** -0.5)[:, 0]
        assert_close(out[b], fb, what=f"bits {bits} D={D} b={b}")
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, D ** -0.5), what=f"bits {bits} b={b}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_rows_other_token_dtypes(dtype):
    # fp32 tokens take the one-row append kernel, bf16 the row4 kernel; the
    # rows must be those of the INT4 cache of the same tokens, packed dense
    rng = np.random.default_rng(11)
    B, H, T, D = 2, 3, 333, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float32)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float32)
    params = dict(stride_k=16, stride_v=8, bits_k=2, bits_v=3, dz_v=0.05, dtype=dtype)
    a = dense_cache(k, v, **params, chunks=[100, 233])
    b = dense_cache(k, v, **params, chunks=[100, 233], dense=False)
    from chronoquant_mlx_amd.persist import dense_pack
    for i, fb in ((2, 2), (4, 3)):
        want = dense_pack(b.state[i], D, fb)
        assert torch.equal(a.state[i].contiguous().view(torch.uint8), want)
    for i in (0, 1, 3, 5):
        assert torch.equal(a.state[i].view(torch.int16), b.state[i].view(torch.int16))


def test_dense_streaming_one_token_per_sequence_offsets():
    # one token per step through per-sequence device offsets (the decode
    # loop's append), then the balanced-plan decode over ragged lengths
    from chronoquant_mlx_amd import ChronoQuantCache
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    rng = np.random.default_rng(12)
    B, H, G, D, T = 3, 8, 4, 128, 1200
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8, bits_k=4, bits_v=3, dz_v=0.05)
    lens = [700, 1100, 450]
    cache = ChronoQuantCache(stride_k=32, stride_v=8, delta_bits_k=4, delta_bits_v=3,
                             dead_zone_v=0.05, dense_residuals=True)
    kt, vt = to_gpu(k), to_gpu(v)
    cache.update_and_fetch(kt[:, :, :400], vt[:, :, :400])
    pos = torch.full((B,), 400, dtype=torch.int32, device="cuda")
    cache.bind_device_position(pos, T)
    for s in range(400, max(lens)):
        cache.update_and_fetch(kt[:, :, s:s + 1], vt[:, :, s:s + 1])
        pos += 1
        cache.advance(1)
    cache.bind_device_position(None)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, D ** -0.5,
                                        seq_lens=seq_lens).float().cpu().numpy()
    for b in range(B):
        ck, cv = build_oracle(k[b, :, :lens[b]], v[b, :, :lens[b]], **params)
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, D ** -0.5), what=f"ragged b={b}")


def test_dense_state_and_persist_round_trips(tmp_path):
    from chronoquant_mlx_amd import ChronoQuantCache, load_prompt_cache, save_prompt_cache
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    rng = np.random.default_rng(13)
    B, H, G, D, T = 2, 4, 4, 128, 500
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = to_gpu(rng.standard_normal((B, G * H, D)))
    params = dict(stride_k=64, stride_v=32, bits_k=4, bits_v=3, dz_v=0.05)
    a = dense_cache(k, v, **params)
    ref = chronoquant_sdpa_cache_kernel(q, a, D ** -0.5)
    # the reference's INT4 state list given to a dense cache is packed dense
    i4 = dense_cache(k, v, **params, dense=False)
    c = ChronoQuantCache(stride_k=64, stride_v=32, delta_bits_v=3, dead_zone_v=0.05,
                         dense_residuals=True)
    c.state = i4.state
    assert all(torch.equal(x, y) for x, y in zip(c.state, a.state))
    for dense_file in (False, True):
        f = str(tmp_path / f"d{int(dense_file)}.safetensors")
        save_prompt_cache(f, [a, i4], dense=dense_file)
        la, li = load_prompt_cache(f)
        assert la.dense_residuals and not li.dense_residuals
        assert all(torch.equal(x, y) for x, y in zip(la.state, a.state))
        assert all(torch.equal(x, y) for x, y in zip(li.state, i4.state))
        assert torch.equal(chronoquant_sdpa_cache_kernel(q, la, D ** -0.5), ref)
        la.update_and_fetch(to_gpu(k[:, :, :7]), to_gpu(v[:, :, :7]))  # appends continue
        assert la.offset == T + 7


def test_dense_prefill_takes_the_reconstruct_fallback():
    from chronoquant_mlx_amd import chronoquant_sdpa
    rng = np.random.default_rng(14)
    B, H, G, D, T, L = 1, 2, 4, 128, 600, 64
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, L, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8, bits_k=4, bits_v=3, dz_v=0.05)
    cache = dense_cache(k, v, **params)
    out = chronoquant_sdpa(to_gpu(q), None, None, cache, D ** -0.5, mask="causal")
    ck, cv = build_oracle(k[0], v[0], **params)
    fb = O.sdpa_fallback(q[0], ck.reconstruct(), cv.reconstruct(), D ** -0.5, causal=True)
    assert_close(out[0].float().cpu().numpy(), fb, what="dense prefill")
