"""Pins the oracle's INT4 packing (reference kernels.py:9-22, 34-61) — CPU only.

The layout is fixed by the MSL pack kernel: word w = sum_i nibble(8w+i) << 4i
with nibble = clip(code + 8, 0, 15), so little-endian byte b of word w holds
dim 8w+2b in its low nibble and dim 8w+2b+1 in its high nibble.
"""
import itertools

import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O


def test_every_nibble_at_every_position():
    # brute force: all 16 codes x 8 positions, other dims at code 0 (nibble 8)
    for code, pos in itertools.product(range(-8, 8), range(8)):
        c = np.zeros((1, 8), np.int8)
        c[0, pos] = code
        w = int(O.pack_int4(c)[0, 0])
        expect = 0
        for i in range(8):
            expect |= ((code + 8) if i == pos else 8) << (4 * i)
        assert w == expect
        assert int(N.pack_int4_codes(c)[0, 0]) == expect


def test_byte_layout_little_endian():
    c = np.array([[-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7]], np.int8)
    w = O.pack_int4(c)
    assert w.tolist() == [[0x76543210, 0xFEDCBA98]]
    b = w.view(np.uint8).reshape(-1).tolist()
    assert b == [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]


def test_out_of_range_codes_clip():
    c = np.array([[-100, 100, -9, 8, 0, 0, 0, 0]], np.int8)
    assert O.pack_int4(c)[0, 0] == 0x8888F0F0  # nibbles 0, 15, 0, 15, 8, 8, 8, 8
    assert N.pack_int4_codes(c)[0, 0] == 0x8888F0F0


@pytest.mark.parametrize("D", [1, 5, 8, 72, 100, 128, 256])
def test_roundtrip_and_pad(D):
    # mirrors tests/test_chronoquant_mlx.py:51-58 (unpack(pack(c)) == c) plus the
    # pad rule: dims past D hold nibble 0
    rng = np.random.default_rng(D)
    c = rng.integers(-8, 8, size=(2, 3, 5, D)).astype(np.int8)
    p = O.pack_int4(c)
    assert p.shape == (2, 3, 5, (D + 7) // 8)
    assert np.array_equal(O.unpack_int4(p, D), c)
    assert np.array_equal(p, N.pack_int4_codes(c))
    assert np.array_equal(N.unpack_int4_codes(p, D), c)
    if D % 8:
        last = p[..., -1]
        used = D % 8
        assert np.all((last >> (4 * used)) == 0)
