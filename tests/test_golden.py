"""The CPU restatements against the committed golden vectors (tests/golden).

Both the C oracle and the numpy restatement must reproduce every fixture bit
for bit: codec codes/scales/packed words, cache state after append, the
reconstruction, and the fallback attention output (fp16); the fused-kernel
output (fp32) to 1e-6 relative.  Closed-form checks that do not depend on
either restatement ride along: unpack(packed) == codes, nibble = code + 8,
and |delta - code * scale| <= scale / 2 outside the clipped and degenerate
rows.
"""
import os

import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
ATTN = ["c0_small", "ft_v3_gqa", "bits3_dz02", "d72", "stride1"]


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def case(g, name):
    H, nq, T, D, sk, sv, bk, bv = (int(x) for x in g[f"{name}/params"])
    dzk, dzv = (float(x) for x in g[f"{name}/dead_zone"])
    return dict(H=H, nq=nq, T=T, D=D, sk=sk, sv=sv, bk=bk, bv=bv, dzk=dzk, dzv=dzv)


def u16(x):
    return np.ascontiguousarray(x).view(np.uint16)


@pytest.mark.parametrize("name", ATTN)
def test_append_state_c_oracle(g, name):
    c = case(g, name)
    for comp, s, b, dz in (("k", c["sk"], c["bk"], c["dzk"]), ("v", c["sv"], c["bv"], c["dzv"])):
        oc = O.OracleComponent(c["H"], c["D"], s, b, dz, capacity=c["T"])
        oc.append(g[f"{name}/{comp}"])
        kf, pk, sc = oc.active()
        assert np.array_equal(u16(kf), u16(g[f"{name}/keyframes_{comp}"]))
        assert np.array_equal(pk, g[f"{name}/packed_{comp}"])
        assert np.array_equal(u16(sc), u16(g[f"{name}/scales_{comp}"]))
        # I-frames reproduce the input exactly (cache.py:103-105)
        x = g[f"{name}/{comp}"]
        assert np.array_equal(u16(kf), u16(x[:, ::s]))


@pytest.mark.parametrize("name", ATTN)
def test_append_state_numpy_restatement(g, name):
    c = case(g, name)
    for comp, s, b, dz in (("k", c["sk"], c["bk"], c["dzk"]), ("v", c["sv"], c["bv"], c["dzv"])):
        nc = N.Component(c["H"], c["D"], s, b, dz)
        nc.append(g[f"{name}/{comp}"].astype(np.float32))
        assert np.array_equal(u16(nc.keyframes), u16(g[f"{name}/keyframes_{comp}"]))
        assert np.array_equal(nc.packed, g[f"{name}/packed_{comp}"])
        assert np.array_equal(u16(nc.scales), u16(g[f"{name}/scales_{comp}"]))


@pytest.mark.parametrize("name", ATTN)
def test_attention_outputs(g, name):
    c = case(g, name)
    ck = O.OracleComponent(c["H"], c["D"], c["sk"], c["bk"], c["dzk"], capacity=c["T"])
    cv = O.OracleComponent(c["H"], c["D"], c["sv"], c["bv"], c["dzv"], capacity=c["T"])
    ck.append(g[f"{name}/k"])
    cv.append(g[f"{name}/v"])
    q = g[f"{name}/q"]
    scale = c["D"] ** -0.5
    fb = O.sdpa_fallback(q[:, None], ck.reconstruct(), cv.reconstruct(), scale)[:, 0]
    assert np.array_equal(u16(fb), u16(g[f"{name}/out_fallback"]))
    fused = O.sdpa_fused(q, ck, cv, scale)
    np.testing.assert_allclose(fused, g[f"{name}/out_fused"], rtol=1e-6, atol=1e-7)
    # the fused semantics and the fallback describe the same attention
    ref = g[f"{name}/out_fallback"].astype(np.float64)
    assert np.max(np.abs(fused - ref)) <= 2e-3 + 1e-2 * np.max(np.abs(ref))


@pytest.mark.parametrize("name", ATTN)
def test_packed_layout_closed_form(g, name):
    """Word w holds dims 8w..8w+7, dim 8w+i at bits 4i (kernels.py:15-21):
    decode the fixture's words by hand and re-encode the reconstruction."""
    c = case(g, name)
    for comp in ("k", "v"):
        pk = g[f"{name}/packed_{comp}"].astype(np.uint64)
        if pk.shape[1] == 0:  # stride 1: no P-frames
            continue
        nib = (pk[..., :, None] >> (4 * np.arange(8, dtype=np.uint64))) & 15
        nib = nib.reshape(pk.shape[:-1] + (-1,))
        D = c["D"]
        assert np.all(nib[..., D:] == 0)  # padding nibble 0 (kernels.py:41-43)
        codes = nib[..., :D].astype(np.int64) - 8
        bits = c["bk"] if comp == "k" else c["bv"]
        assert codes.min() >= -(2 ** bits // 2) and codes.max() <= 2 ** bits // 2 - 1
        assert np.array_equal(O.unpack_int4(g[f"{name}/packed_{comp}"], D), codes)


def test_codec_vectors(g):
    d = g["codec/delta"]
    for bits in (4, 3):
        for dz in (0.0, 0.2):
            tag = f"codec/b{bits}_dz{int(dz * 10)}"
            c, s = O.quantize_delta(d, bits, dz)
            assert np.array_equal(c, g[tag + "_codes"]), tag
            assert np.array_equal(u16(s), u16(g[tag + "_scales"])), tag
            cn, sn = N.quantize_delta(d.astype(np.float32), bits, dz)
            assert np.array_equal(cn, g[tag + "_codes"]), tag
            assert np.array_equal(u16(sn.reshape(s.shape)), u16(g[tag + "_scales"])), tag
            assert np.array_equal(O.pack_int4(c), g[tag + "_packed"]), tag
            # nibble = code + 8 at bits 4i of the row's single word
            w = g[tag + "_packed"][:, 0].astype(np.uint64)
            for i in range(8):
                assert np.array_equal(((w >> (4 * i)) & 15).astype(np.int64), c[:, i] + 8)


def test_codec_vectors_closed_form(g):
    """Rows whose codes follow from the IEEE rules alone."""
    d = g["codec/delta"]
    c4, s4 = g["codec/b4_dz0_codes"], g["codec/b4_dz0_scales"]
    # row 0: A = 0.875, s = 0.125 exactly, q = d / s exact, ties to even
    assert float(s4[0]) == 0.125
    assert c4[0].tolist() == [7, 2, 4, -2, 0, 2, 0, -2]
    # row 2: A = 2^-24, s = fp16(2^-24 / 7) = 0 -> +-inf -> clipped
    assert float(s4[2]) == 0.0 and c4[2, :3].tolist() == [7, -8, 0]
    # row 3: A = 0 -> 0/0 -> defined code 0
    assert float(s4[3]) == 0.0 and np.all(c4[3] == 0)
    # row 5: one-hot 3.0 -> s = fp16(3/7), code 7 at the hot dim, 0 elsewhere
    assert float(s4[5]) == float(np.float16(3.0 / 7.0))
    assert c4[5].tolist() == [0, 0, 7, 0, 0, 0, 0, 0]
    # |d - c s| <= s/2 + the fp16 rounding of q = d/s (|q| <= 7: 7 * 2^-11 s)
    # where nothing clips (rows 0, 4, 5, 6)
    for r in (0, 4, 5, 6):
        s = float(s4[r])
        err = np.abs(d[r].astype(np.float64) - c4[r] * s)
        assert np.all(err <= s / 2 + 7 * 2.0 ** -11 * s), r
    # dead zone 0.2 zeroes |d| < fp16(0.7 * 0.2) in row 6 and keeps A' = 0.7,
    # so the scale is unchanged; dim 0 (0.1, code 1 without the dead zone)
    # becomes 0, dim 7 (-0.15) survives
    c4z, s4z = g["codec/b4_dz2_codes"], g["codec/b4_dz2_scales"]
    assert float(s4z[6]) == float(s4[6])
    assert c4[6, 0] == 1 and c4z[6, 0] == 0
    assert c4z[6, 7] == c4[6, 7] != 0
    # 3-bit range [-4, 3]
    c3 = g["codec/b3_dz0_codes"]
    assert c3.min() >= -4 and c3.max() <= 3
