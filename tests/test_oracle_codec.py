"""Pins the CPU oracle's codec (reference codec.py:23-65) — CPU only.

Known-answer rows below were worked out by hand from IEEE binary16 rounding;
each comment shows the arithmetic.  Both restatements (C: oracle/cq_oracle.c,
numpy: oracle/np_oracle.py) must produce them, and must agree bit for bit on
random rows of every dtype / bit width / dead zone.
"""
import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O


def both(delta, bits, dz, dtype="f16"):
    c1, s1 = O.quantize_delta(np.asarray(delta, np.float16 if dtype == "f16" else np.float32),
                              bits, dz, dtype)
    c2, s2 = N.quantize_delta(np.asarray(delta, np.float32), bits, dz, dtype)
    assert np.array_equal(c1, c2)
    assert np.array_equal(s1.view(np.uint16), s2[..., 0].view(np.uint16))
    return c1, s1.astype(np.float32)


def row(*vals, D=16):
    r = np.zeros((1, D), np.float32)
    r[0, : len(vals)] = vals
    return r


def test_half_even_ties():
    # amax = 0.875 -> s = 0.875/7 = 0.125 exactly; q = d/s exact:
    # 0.3125 -> 2.5 -> 2, 0.4375 -> 3.5 -> 4, -0.3125 -> -2.5 -> -2,
    # 0.0625 -> 0.5 -> 0, 0.1875 -> 1.5 -> 2, -0.0625 -> -0, -0.1875 -> -2
    c, s = both(row(0.875, 0.3125, 0.4375, -0.3125, 0.0625, 0.1875, -0.0625, -0.1875), 4, 0.0)
    assert s[0] == 0.125
    assert c[0, :8].tolist() == [7, 2, 4, -2, 0, 2, 0, -2]
    assert not c[0, 8:].any()


def test_quotient_rounded_to_fp16_before_rint():
    # s = fp16(1/7) = 1170 * 2^-13 = 0.142822265625
    # d = 0.499755859375 (2047 * 2^-12): d/s = 3.49914.. -> fp16 3.5 -> rint -> 4
    # (rounding the exact quotient would give 3)
    c, s = both(row(1.0, 0.499755859375), 4, 0.0)
    assert s[0] == np.float32(0.142822265625)
    assert c[0, :2].tolist() == [7, 4]


def test_three_bit_range():
    # 3 bits: half_levels 4, s = amax/3; amax = 0.75 -> s = 0.25
    # 0.375 -> 1.5 -> 2; -0.75 -> -3; 0.625 -> 2.5 -> 2; 0.125 -> 0.5 -> 0
    c, s = both(row(0.75, 0.375, -0.75, 0.625, 0.125), 3, 0.0)
    assert s[0] == 0.25
    assert c[0, :5].tolist() == [3, 2, -3, 2, 0]


def test_two_bit_range():
    # 2 bits: half_levels 2, s = amax/1; codes clip to [-2, 1]
    c, s = both(row(0.5, -0.5, 0.25, -0.25, 0.3), 2, 0.0)
    # 0.25/0.5 = 0.5 -> 0; -0.25/0.5 -> -0; 0.3 fp16 0.2998046875/0.5 -> 0.5996 -> 1
    assert s[0] == 0.5
    assert c[0, :5].tolist() == [1, -1, 0, 0, 1]


def test_dead_zone_zeroes_small_residuals():
    # amax = 0.875, s = 0.125; fp16(0.2) = 0.199951171875,
    # thr = fp16(0.875 * 0.199951171875 = 0.17495727..) = 0.1749267578125
    # 0.150146484375 < thr -> 0 (without dz: 1.2 -> 1); 0.1875 >= thr -> 1.5 -> 2
    c0, _ = both(row(0.875, 0.150146484375, 0.1875), 4, 0.0)
    c1, s1 = both(row(0.875, 0.150146484375, 0.1875), 4, 0.2)
    assert c0[0, :3].tolist() == [7, 1, 2]
    assert c1[0, :3].tolist() == [7, 0, 2]
    assert s1[0] == 0.125


def test_dead_zone_below_half_step_is_a_noop():
    # dz < 0.5/(h-1) only zeroes values whose code is already 0
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4000, 128)) * rng.lognormal(0, 1, (4000, 1))).astype(np.float16)
    for bits, dz in ((4, 0.05), (4, 0.07), (3, 0.05), (3, 0.16)):
        a, sa = O.quantize_delta(x, bits, 0.0)
        b, sb = O.quantize_delta(x, bits, dz)
        assert np.array_equal(a, b) and np.array_equal(sa.view(np.uint16), sb.view(np.uint16))


def test_all_zero_row_fp16_is_code_zero():
    # amax = 0 -> s = 0; fp16(1e-10) == 0 so the guards never fire; 0/0 = NaN -> code 0
    c, s = both(row(), 4, 0.0)
    assert s[0] == 0.0 and not c.any()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_all_zero_row_guarded_dtypes(dtype):
    # bf16/fp32 represent 1e-10, so scale < eps -> scale_safe 1, codes forced 0
    c, s = both(row(), 4, 0.0, dtype)
    assert s[0] == 0.0 and not c.any()


def test_scale_underflow_fp16():
    # amax = 2^-24 (smallest subnormal): s = fp16(2^-24/7) = 0 (below 2^-25)
    # d/0 = +inf -> clip 7, -inf -> clip -8, 0/0 -> NaN -> 0
    tiny = float(np.float16(2.0 ** -24))
    c, s = both(row(tiny, -tiny, 0.0), 4, 0.0)
    assert s[0] == 0.0
    assert c[0, :3].tolist() == [7, -8, 0]


def test_one_hot_row():
    c, s = both(row(0.0, 0.0, -3.0, 0.0), 4, 0.0)
    assert c[0, :4].tolist() == [0, 0, -7, 0]
    assert s[0] == np.float16(3.0 / 7)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("bits,dz", [(4, 0.0), (3, 0.05), (4, 0.2), (2, 0.3), (3, 0.5)])
def test_c_and_numpy_restatements_agree(dtype, bits, dz):
    rng = np.random.default_rng(bits * 100 + int(dz * 10))
    x = (rng.standard_normal((3000, 128)) * rng.lognormal(0, 1.5, (3000, 1))).astype(np.float32)
    if dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
    elif dtype == "bf16":
        x = N.bf16_bits_to_f32(N.f32_to_bf16_bits(x))
    both(x, bits, dz, dtype)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_error_bound_invariant(bits):
    # |d - c*s| <= s/2 up to the fp16 rounding of d/s (relative 2^-11)
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal((2000, 128)) * rng.lognormal(0, 1, (2000, 1))).astype(np.float16)
    c, s = O.quantize_delta(x, bits, 0.0)
    s = s.astype(np.float64)[:, None]
    err = np.abs(x.astype(np.float64) - c * s)
    half = (2 ** bits) // 2
    assert c.max() <= half - 1 and c.min() >= -half
    assert np.all(err <= s * (0.5 + 2.0 ** -10 * (half + 1)) + 1e-12)


def test_oracle_conversions_match_numpy():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, size=400_000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    ok = ~np.isnan(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(f)[ok], ref[ok])
    allh = np.arange(65536, dtype=np.uint16)
    back = O.f16_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    m = ~np.isnan(ref)
    assert np.array_equal(back[m].view(np.uint32), ref[m].view(np.uint32))
    assert np.array_equal(O.f32_to_bf16(f)[ok], N.f32_to_bf16_bits(f)[ok])
