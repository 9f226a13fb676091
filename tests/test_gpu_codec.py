"""GPU parity of the codec, packing, append and reconstruction kernels
(bit exact against the CPU oracle).  Calls go through libchronoquant.so."""
import numpy as np
import pytest
import torch

from oracle import np_oracle as N
from oracle import oracle as O
from tests.cqtest import assert_state_equal, build_gpu_cache, build_oracle, to_gpu

pytestmark = pytest.mark.gpu

TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def gpu_quantize(x: np.ndarray, bits, dz, dtype="f16"):
    from chronoquant_mlx_amd.codec import ChronoQuantCodec
    codec = ChronoQuantCodec(delta_bits=bits, dead_zone_ratio=dz, log_interval=0)
    if dtype == "bf16":
        t = torch.from_numpy(N.f32_to_bf16_bits(x).view(np.int16)).cuda().view(torch.bfloat16)
    else:
        t = to_gpu(x, TORCH_DT[dtype])
    c, s = codec.quantize_delta(t)
    return c.cpu().numpy(), s[..., 0].cpu().numpy()


def test_known_answer_rows():
    rows = np.zeros((6, 16), np.float32)
    rows[0, :8] = [0.875, 0.3125, 0.4375, -0.3125, 0.0625, 0.1875, -0.0625, -0.1875]
    rows[1, :2] = [1.0, 0.499755859375]
    rows[2, :3] = [2.0 ** -24, -(2.0 ** -24), 0.0]
    rows[4, :4] = [0.0, 0.0, -3.0, 0.0]
    rows[5, :3] = [0.875, 0.150146484375, 0.1875]
    c, s = gpu_quantize(rows, 4, 0.0)
    assert c[0, :8].tolist() == [7, 2, 4, -2, 0, 2, 0, -2] and s[0] == 0.125
    assert c[1, :2].tolist() == [7, 4]
    assert c[2, :3].tolist() == [7, -8, 0] and s[2] == 0
    assert not c[3].any() and s[3] == 0
    assert c[4, :4].tolist() == [0, 0, -7, 0]
    assert c[5, :3].tolist() == [7, 1, 2]
    c, _ = gpu_quantize(rows[5:6], 4, 0.2)
    assert c[0, :3].tolist() == [7, 0, 2]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("bits,dz", [(4, 0.0), (3, 0.05), (4, 0.2), (2, 0.3)])
@pytest.mark.parametrize("D", [128, 64, 256, 72, 5])
def test_quantize_matches_oracle(dtype, bits, dz, D):
    rng = np.random.default_rng(D * 7 + bits)
    x = (rng.standard_normal((777, D)) * rng.lognormal(0, 1.5, (777, 1))).astype(np.float32)
    if dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
    elif dtype == "bf16":
        x = N.bf16_bits_to_f32(N.f32_to_bf16_bits(x))
    x[3] = 0.0  # an all-zero row
    c_g, s_g = gpu_quantize(x, bits, dz, dtype)
    c_o, s_o = O.quantize_delta(x.astype(np.float16) if dtype == "f16" else x, bits, dz, dtype)
    bad = np.argwhere(c_g != c_o)
    assert bad.size == 0, f"{len(bad)} codes differ, first {bad[:4].tolist()}"
    assert np.array_equal(s_g.view(np.uint16), s_o.view(np.uint16))


@pytest.mark.parametrize("D", [1, 5, 8, 72, 128, 256])
def test_pack_unpack_match_oracle(D):
    from chronoquant_mlx_amd.kernels import pack_int4_codes, unpack_int4_codes
    rng = np.random.default_rng(D)
    c = rng.integers(-8, 8, size=(3, 4, 33, D)).astype(np.int8)
    p = pack_int4_codes(torch.from_numpy(c).cuda())
    assert np.array_equal(p.cpu().numpy(), O.pack_int4(c))
    u = unpack_int4_codes(p, D)
    assert np.array_equal(u.cpu().numpy(), c)


CASES = [
    # (stride_k, stride_v, bits_k, bits_v, dz_k, dz_v, D)
    (32, 8, 4, 4, 0.0, 0.0, 128),     # c0/c1 standard
    (64, 32, 4, 3, 0.0, 0.05, 128),   # c2 Full-Throttle V3
    (32, 8, 4, 4, 0.0, 0.05, 128),    # reference defaults
    (1, 3, 4, 2, 0.0, 0.3, 64),       # stride 1 (no K P-frames), 2-bit
    (5, 7, 3, 4, 0.2, 0.0, 72),       # D % 8 != 0 pad path, active dead zone
    (16, 16, 4, 4, 0.0, 0.0, 256),
]


@pytest.mark.parametrize("case", CASES)
def test_append_bulk_matches_oracle(case):
    sk, sv, bk, bv, dzk, dzv, D = case
    rng = np.random.default_rng(sk * 31 + D)
    B, H, T = 2, 4, 333
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    params = dict(stride_k=sk, stride_v=sv, bits_k=bk, bits_v=bv, dz_k=dzk, dz_v=dzv)
    cache = build_gpu_cache(k, v, **params)
    for b in range(B):
        assert_state_equal(cache, b, *build_oracle(k[b], v[b], **params))


@pytest.mark.parametrize("H,chunks", [(3, None), (3, [1, 2, 100, 7, 1, 222]), (5, [37, 1, 295])])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_append_rows_straddle_components(H, chunks, dtype):
    # Head_dim 128 appends with 16-bit tokens encode four rows per wave
    # (append_row4_kernel).  With B*S*H odd a wave's rows straddle the K / V
    # boundary and mix I-frames, anchors appended by the same call and
    # anchors already in the cache; odd chunk sizes move every boundary.
    rng = np.random.default_rng(H * 7 + len(chunks or []))
    B, T, D = 1, 333, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.2, axis=2).astype(np.float32)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.2, axis=2).astype(np.float32)
    if dtype == "bf16":
        k = N.bf16_bits_to_f32(N.f32_to_bf16_bits(k))
        v = N.bf16_bits_to_f32(N.f32_to_bf16_bits(v))
    else:
        k, v = k.astype(np.float16), v.astype(np.float16)
    params = dict(stride_k=64, stride_v=32, bits_k=4, bits_v=3, dz_v=0.05)
    cache = build_gpu_cache(k, v, chunks=chunks, dtype=TORCH_DT[dtype], **params)
    assert_state_equal(cache, 0, *build_oracle(k[0], v[0], dtype=dtype, **params))


@pytest.mark.parametrize("device_pos", [False, True])
def test_append_strided_rows_take_the_one_row_path(device_pos):
    # Rows that do not start 16-byte aligned (a head_dim-128 slice of wider
    # rows) go through append_kernel instead of the four-row kernel: the
    # same cache state.  B * H = 9 rows per token, so the four-row kernel's
    # waves also straddle sequences; with device positions the sequences
    # append at different offsets (sequences 1 and 2 rewrite earlier ones).
    from chronoquant_mlx_amd import ChronoQuantCache
    g = torch.Generator(device="cuda").manual_seed(5)
    B, H, T, D = 3, 3, 200, 128
    wide = torch.randn(2, B, H, T, D + 4, device="cuda", generator=g).half()
    k, v = wide[0, ..., :D], wide[1, ..., :D]
    assert k.stride(2) % 8 != 0
    caches = []
    for kk, vv in ((k, v), (k.contiguous(), v.contiguous())):
        c = ChronoQuantCache(stride_k=32, stride_v=8, dead_zone_v=0.05)
        c.update_and_fetch(kk[:, :, :77], vv[:, :, :77])
        if device_pos:
            pos = torch.tensor([77, 70, 61], dtype=torch.int32, device="cuda")
            c.bind_device_position(pos, T)
            for s0 in range(77, T, 41):  # multi-token appends at per-sequence offsets
                s1 = min(s0 + 41, T)
                c.update_and_fetch(kk[:, :, s0:s1], vv[:, :, s0:s1])
                pos += s1 - s0
        else:
            c.update_and_fetch(kk[:, :, 77:], vv[:, :, 77:])
        caches.append(c)
    if not device_pos:
        for a, b in zip(caches[0].state, caches[1].state):
            assert torch.equal(a, b)
        return
    # every written row: sequence b holds positions [0, T - shift_b)
    from chronoquant_mlx_amd.cache import _num_keyframes, _num_pframes
    for b, top in enumerate((T, T - 7, T - 16)):
        for comp in ("k", "v"):
            s = caches[0]._stride(comp)
            nk, npf = _num_keyframes(top, s), _num_pframes(top, s)
            for arr, n in ((caches[0]._kf, nk), (caches[0]._pk, npf), (caches[0]._sc, npf)):
                other = {id(caches[0]._kf): caches[1]._kf, id(caches[0]._pk): caches[1]._pk,
                         id(caches[0]._sc): caches[1]._sc}[id(arr)]
                x, y = arr[comp][b, :, :n], other[comp][b, :, :n]
                assert torch.equal(x.view(torch.int16) if x.element_size() == 2 else x.view(torch.int32),
                                   y.view(torch.int16) if y.element_size() == 2 else y.view(torch.int32)), \
                    (b, comp)


def test_append_streaming_equals_bulk():
    rng = np.random.default_rng(9)
    B, H, T, D = 1, 8, 300, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    params = dict(stride_k=32, stride_v=8)
    bulk = build_gpu_cache(k, v, **params)
    chunks = [1, 1, 30, 2, 64, 1, 100, 101]
    stream = build_gpu_cache(k, v, chunks=chunks, **params)
    one = build_gpu_cache(k, v, chunks=[1] * T, **params)
    for a, b, c in zip(bulk.state, stream.state, one.state):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert bulk.nbytes == stream.nbytes == one.nbytes


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_append_non_fp16_inputs(dtype):
    rng = np.random.default_rng(4)
    B, H, T, D = 1, 4, 200, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.2, axis=2).astype(np.float32)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.2, axis=2).astype(np.float32)
    if dtype == "bf16":
        k = N.bf16_bits_to_f32(N.f32_to_bf16_bits(k))
        v = N.bf16_bits_to_f32(N.f32_to_bf16_bits(v))
    params = dict(stride_k=32, stride_v=8, dz_v=0.05)
    cache = build_gpu_cache(k, v, dtype=TORCH_DT[dtype], **params)
    assert_state_equal(cache, 0, *build_oracle(k[0], v[0], dtype=dtype, **params))


def test_append_c0_full_and_reconstruct():
    from chronoquant_mlx_amd import synth
    cfg = synth.CONFIGS["c0"]
    k, v = synth.make_kv(cfg)
    params = dict(stride_k=cfg.stride_k, stride_v=cfg.stride_v)
    cache = build_gpu_cache(k, v, chunks=[1000, 1, 3095], **params)
    ck, cv = build_oracle(k[0], v[0], **params)
    assert_state_equal(cache, 0, ck, cv)
    rk, rv = cache.reconstruct_history()
    assert np.array_equal(rk[0].cpu().numpy().view(np.uint16), ck.reconstruct().view(np.uint16))
    assert np.array_equal(rv[0].cpu().numpy().view(np.uint16), cv.reconstruct().view(np.uint16))
    # the reference's nbytes for c0: 5,298,176 bytes
    assert cache.nbytes == synth.compressed_bytes(cfg.T, 8, 128, 32, 8) == 5298176


def test_state_roundtrip():
    from chronoquant_mlx_amd import ChronoQuantCache
    rng = np.random.default_rng(12)
    k = rng.standard_normal((1, 2, 77, 128)).astype(np.float16)
    v = rng.standard_normal((1, 2, 77, 128)).astype(np.float16)
    a = build_gpu_cache(k, v, stride_k=1, stride_v=8)
    assert len(a.state) == 6 and a.state[2].shape[2] == 0
    b = ChronoQuantCache(stride_k=1, stride_v=8)
    b.state = [t.clone() for t in a.state]
    assert b.offset == 77
    for x, y in zip(a.state, b.state):
        assert torch.equal(x, y)
    # appending after a restore continues the stream identically
    nk = to_gpu(rng.standard_normal((1, 2, 5, 128)).astype(np.float16))
    a.update_and_fetch(nk, nk)
    b.update_and_fetch(nk, nk)
    for x, y in zip(a.state, b.state):
        assert torch.equal(x, y)
