"""Generate the committed golden vectors of the ChronoQuant hot path.

The reference ships no golden vectors, known-answer tests or fixtures for this
path (its tests compare MLX with MLX under tolerances), and MLX is not
importable here, so these vectors come from the two CPU restatements of the
reference algorithm: the C oracle (oracle/cq_oracle.c) and the independent
numpy restatement (oracle/np_oracle.py).  The generator refuses to write a
case on which the two disagree.  The committed file freezes both against
drift, and the GPU tests compare the HIP path with it.

Cases (the fixture list of the reference's codec, cache and attention files):
  c0_small    configs[0] parameters (strides 32/8, INT4/INT4, dz 0, MHA) at
              2 kv heads x 64 tokens            codec.py:23-65, cache.py:87-156
  ft_v3_gqa   Full-Throttle V3 (64/32, K 4-bit, V 3-bit, dz_v 0.05), GQA 4,
              2 kv heads x 96 tokens             patch.py:81-88
  bits3_dz02  3-bit codes with dead zone 0.2 (above the no-op threshold)
              on both components, strides 4/4    codec.py:36-45
  d72         head_dim 72: the pack's padding nibble   kernels.py:41-43
  stride1     stride_k 1 (K all I-frames)        cache.py:53-61
  codec_*     hand-built deltas: exact .5 ties, all-equal |d|, all-zero,
              an underflowing scale, one-hot, a double-rounding row; at
              4 and 3 bits, dead zone 0 and 0.2
Each attention case stores q, the fallback output (attention.py:61-74,
fp16) and the fused-kernel output (kernels.py:79-228, fp32).

    python tests/golden/make_golden.py     # rewrites tests/golden/golden.npz
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import np_oracle as N  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")

# (name, H, nq, T, D, stride_k, stride_v, bits_k, bits_v, dz_k, dz_v, seed)
ATTN_CASES = [
    ("c0_small", 2, 2, 64, 128, 32, 8, 4, 4, 0.0, 0.0, 11),
    ("ft_v3_gqa", 2, 8, 96, 128, 64, 32, 4, 3, 0.0, 0.05, 12),
    ("bits3_dz02", 2, 2, 40, 128, 4, 4, 3, 3, 0.2, 0.2, 13),
    ("d72", 2, 4, 50, 72, 16, 4, 4, 4, 0.0, 0.0, 14),
    ("stride1", 2, 2, 24, 128, 1, 8, 4, 4, 0.0, 0.0, 15),
]


def ar1(H, T, D, seed):
    """Seeded AR(1) fp16 stream [H, T, D] with per-channel log-normal scale."""
    rng = np.random.default_rng(seed)
    sig = rng.lognormal(0.0, 0.5, size=(H, D))
    x = rng.normal(0.0, 0.2 / np.sqrt(1 - 0.98 ** 2), size=(H, D))
    out = np.empty((H, T, D), np.float16)
    for t in range(T):
        if t:
            x = 0.98 * x + 0.2 * rng.standard_normal((H, D))
        out[:, t] = (sig * x).astype(np.float16)
    return out


def codec_rows():
    """Hand-built delta rows (D = 8) covering the codec's special cases."""
    rows = [
        [0.875, 0.3125, 0.4375, -0.1875, 0.0, 0.25, 0.0625, -0.3125],  # .5 ties at s=0.125
        [1.0, 0.499755859375, 0, 0, 0, 0, 0, 0],                        # double rounding
        [2.0 ** -24, -(2.0 ** -24), 0, 0, 0, 0, 0, 0],                  # scale underflows to 0
        [0.0] * 8,                                                      # A = 0
        [0.5, -0.5, 0.5, -0.5, 0.5, -0.5, 0.5, -0.5],                   # all-equal |d|
        [0.0, 0.0, 3.0, 0.0, 0.0, 0.0, 0.0, 0.0],                       # one-hot
        [0.1, -0.02, 0.3, 0.05, -0.7, 0.01, 0.2, -0.15],                # dead-zone victims
        [65504.0, -65504.0, 1.0, -1.0, 0.0, 2.0, -3.0, 4.0],            # fp16 max
    ]
    return np.array(rows, np.float16)


def attention_case(name, H, nq, T, D, sk, sv, bk, bv, dzk, dzv, seed):
    k = ar1(H, T, D, seed)
    v = ar1(H, T, D, seed + 1000)
    q = np.random.default_rng(seed + 2000).standard_normal((nq, D)).astype(np.float16)
    scale = D ** -0.5
    ck = O.OracleComponent(H, D, sk, bk, dzk, capacity=T)
    cv = O.OracleComponent(H, D, sv, bv, dzv, capacity=T)
    ck.append(k)
    cv.append(v)
    # the independent numpy restatement must agree bit for bit
    for comp, x, s, b, dz in ((ck, k, sk, bk, dzk), (cv, v, sv, bv, dzv)):
        nc = N.Component(H, D, s, b, dz)
        nc.append(x.astype(np.float32))
        kf, pk, sc = comp.active()
        assert np.array_equal(kf.view(np.uint16), nc.keyframes.view(np.uint16)), name
        assert np.array_equal(pk, nc.packed), name
        assert np.array_equal(sc.view(np.uint16), nc.scales.view(np.uint16)), name
        assert np.array_equal(comp.reconstruct().view(np.uint16),
                              nc.reconstruct().view(np.uint16)), name
    rk, rv = ck.reconstruct(), cv.reconstruct()
    fb = O.sdpa_fallback(q[:, None], rk, rv, scale)[:, 0]
    fb_np = N.sdpa_fallback(q[:, None], rk, rv, scale)[:, 0]
    ulp = np.abs(fb.astype(np.float64) - fb_np.astype(np.float64))
    assert np.all(ulp <= np.spacing(np.abs(fb).astype(np.float16)).astype(np.float64)), name
    fused = O.sdpa_fused(q, ck, cv, scale)
    p = f"{name}/"
    kfk, pkk, sck = ck.active()
    kfv, pkv, scv = cv.active()
    return {
        p + "params": np.array([H, nq, T, D, sk, sv, bk, bv], np.int64),
        p + "dead_zone": np.array([dzk, dzv], np.float64),
        p + "k": k, p + "v": v, p + "q": q,
        p + "keyframes_k": kfk.copy(), p + "packed_k": pkk.copy(), p + "scales_k": sck.copy(),
        p + "keyframes_v": kfv.copy(), p + "packed_v": pkv.copy(), p + "scales_v": scv.copy(),
        p + "out_fallback": fb, p + "out_fused": fused,
    }


def codec_cases():
    d = codec_rows()
    out = {"codec/delta": d}
    for bits in (4, 3):
        for dz in (0.0, 0.2):
            c, s = O.quantize_delta(d, bits, dz)
            cn, sn = N.quantize_delta(d.astype(np.float32), bits, dz)
            assert np.array_equal(c, cn) and np.array_equal(
                s.view(np.uint16), sn.reshape(s.shape).view(np.uint16)), (bits, dz)
            tag = f"codec/b{bits}_dz{int(dz * 10)}"
            out[tag + "_codes"] = c
            out[tag + "_scales"] = s
            out[tag + "_packed"] = O.pack_int4(c)
    return out


def generate():
    O.build()
    data = {}
    for case in ATTN_CASES:
        data.update(attention_case(*case))
    data.update(codec_cases())
    return data


if __name__ == "__main__":
    arrays = generate()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {len(arrays)} arrays, {os.path.getsize(OUT)} bytes")
