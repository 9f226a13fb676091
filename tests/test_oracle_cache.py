"""Pins the oracle's cache state machine (reference cache.py:53-160) — CPU only."""
import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O


@pytest.mark.parametrize("stride", [1, 2, 3, 8, 32, 64])
def test_frame_counts_closed_form(stride):
    for T in range(0, 200):
        nkf = O.num_keyframes(T, stride)
        npf = O.num_pframes(T, stride)
        # brute force over positions: t is an I-frame iff t % stride == 0
        assert nkf == sum(1 for t in range(T) if t % stride == 0)
        assert nkf + npf == T
        # P-frame slot of token t is t - t//stride - 1, dense in [0, npf)
        slots = [t - t // stride - 1 for t in range(T) if t % stride]
        assert slots == list(range(npf))


def _manual_reconstruct(x, stride, delta_bits=4):
    """Restatement of the reference test's own codec (tests/test_chronoquant_mlx.py:15-36),
    in numpy fp16: no dead zone; recon = anchor + fp16(code) * fp16 scale."""
    half = (2 ** delta_bits) // 2
    H, T, D = x.shape
    out, kfs = [], []
    for t in range(T):
        tok = x[:, t, :]
        if t % stride == 0:
            kfs.append(tok.astype(np.float16))
            out.append(kfs[-1])
            continue
        anchor = kfs[t // stride]
        delta = (tok - anchor).astype(np.float16)
        amax = np.abs(delta).max(axis=-1, keepdims=True)
        scale = (amax / np.float16(half - 1)).astype(np.float16)
        with np.errstate(invalid="ignore", divide="ignore"):
            codes = np.rint((delta / scale).astype(np.float16))
        codes = np.clip(np.nan_to_num(codes), -half, half - 1).astype(np.int8)
        rec = (anchor + (codes.astype(np.float16) * scale).astype(np.float16)).astype(np.float16)
        out.append(rec)
    return np.stack(out, axis=1)


def test_reconstruct_matches_reference_test_restatement():
    # the reference's TestCache case: stride 4 (K) / 2 (V), shape (1, 2, 9, 128)
    rng = np.random.default_rng(7)
    for stride in (4, 2):
        x = rng.standard_normal((2, 9, 128)).astype(np.float16)
        c = O.OracleComponent(2, 128, stride, 4, 0.0, capacity=9)
        c.append(x)
        assert np.array_equal(c.reconstruct().view(np.uint16),
                              _manual_reconstruct(x, stride).view(np.uint16))


@pytest.mark.parametrize("stride,bits,dz,D", [(32, 4, 0.0, 128), (8, 4, 0.05, 128),
                                             (64, 4, 0.0, 128), (32, 3, 0.05, 128),
                                             (1, 4, 0.0, 64), (5, 3, 0.2, 72)])
def test_streaming_equals_bulk_and_numpy(stride, bits, dz, D):
    rng = np.random.default_rng(stride + D)
    H, T = 2, 150
    x = np.cumsum(rng.standard_normal((H, T, D)) * 0.1, axis=1).astype(np.float16)
    bulk = O.OracleComponent(H, D, stride, bits, dz, capacity=T)
    bulk.append(x)
    stream = O.OracleComponent(H, D, stride, bits, dz, capacity=T)
    for t in range(T):
        stream.append(x[:, t: t + 1])
    ref = N.Component(H, D, stride, bits, dz)
    ref.append(x.astype(np.float32))
    for a, b in zip(bulk.active(), stream.active()):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    kf, pk, sc = bulk.active()
    assert np.array_equal(kf.view(np.uint16), ref.keyframes.view(np.uint16))
    assert np.array_equal(pk, ref.packed)
    assert np.array_equal(sc.view(np.uint16), ref.scales.view(np.uint16))
    r = bulk.reconstruct()
    assert np.array_equal(r.view(np.uint16), ref.reconstruct().view(np.uint16))
    # I-frames reproduce their tokens exactly (cache.py:104)
    assert np.array_equal(r[:, ::stride].view(np.uint16), x[:, ::stride].view(np.uint16))


def test_reconstruction_error_bound():
    # |x - r| <= s/2 (+ fp16 roundings) per P-frame element
    rng = np.random.default_rng(11)
    H, T, D, s = 2, 256, 128, 8
    x = np.cumsum(rng.standard_normal((H, T, D)) * 0.05, axis=1).astype(np.float16)
    c = O.OracleComponent(H, D, s, 4, 0.0, capacity=T)
    c.append(x)
    r = c.reconstruct().astype(np.float64)
    _, _, sc = c.active()
    err = np.abs(r - x.astype(np.float64))
    pos = np.arange(T)
    pf = pos[pos % s != 0]
    scale = sc.astype(np.float64)[:, pf - pf // s - 1]
    mag = np.abs(x.astype(np.float64))[:, pf]
    assert np.all(err[:, pf] <= scale[..., None] * 0.51 + mag * 2.0 ** -10 + 1e-7)
    assert np.all(err[:, pos % s == 0] == 0)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_non_fp16_inputs_agree_with_numpy(dtype):
    rng = np.random.default_rng(5)
    H, T, D = 2, 70, 128
    x = np.cumsum(rng.standard_normal((H, T, D)) * 0.2, axis=1).astype(np.float32)
    if dtype == "bf16":
        x = N.bf16_bits_to_f32(N.f32_to_bf16_bits(x))
    c = O.OracleComponent(H, D, 8, 4, 0.05, capacity=T)
    c.append(x, dtype)
    ref = N.Component(H, D, 8, 4, 0.05, dtype)
    ref.append(x)
    kf, pk, sc = c.active()
    assert np.array_equal(kf.view(np.uint16), ref.keyframes.view(np.uint16))
    assert np.array_equal(pk, ref.packed)
    assert np.array_equal(sc.view(np.uint16), ref.scales.view(np.uint16))
