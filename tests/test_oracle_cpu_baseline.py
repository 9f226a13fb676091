"""The CPU baseline that bench.py times (oracle/cq_cpu_baseline.c) computes
the reference's fused operator (kernels.py:79-228): its fp32 output matches
the committed golden `out_fused` vectors and the binary64 fused oracle to
fp32 rounding, whatever key split it runs with.

Bar: |d| <= 1e-5 + 1e-4 * absw, absw the softmax-weighted mean of |v| per
element (the scale of a weighted sum's rounding error).  fp32 scores carry
relative error ~T * 2^-24 in the worst case; a dropped keyframe, a wrong
nibble, a wrong anchor or a wrong merge factor moves the output by orders
of magnitude more.
"""
import dataclasses
import os

import numpy as np
import pytest

from chronoquant_mlx_amd import synth
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
ATTN = ["c0_small", "ft_v3_gqa", "bits3_dz02", "d72", "stride1"]


def check(got, ref, absw, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = 1e-5 + 1e-4 * absw.astype(np.float64)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (f"{what}: |d|={err[worst]:.3e} > {bound[worst]:.3e} "
                                  f"at {tuple(int(i) for i in worst)}")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ATTN)
@pytest.mark.parametrize("n_chunks", [0, 1, 3])
def test_baseline_on_golden(g, name, n_chunks):
    H, nq, T, D, sk, sv, bk, bv = (int(x) for x in g[f"{name}/params"])
    dzk, dzv = (float(x) for x in g[f"{name}/dead_zone"])
    ck = O.OracleComponent(H, D, sk, bk, dzk, capacity=T)
    cv = O.OracleComponent(H, D, sv, bv, dzv, capacity=T)
    ck.append(g[f"{name}/k"])
    cv.append(g[f"{name}/v"])
    q = g[f"{name}/q"]
    scale = D ** -0.5
    _, absw = O.sdpa_fused(q, ck, cv, scale, return_absw=True)
    got = O.fused_decode_f32(q, ck, cv, scale, n_chunks=n_chunks)
    check(got, g[f"{name}/out_fused"], absw, f"{name} chunks={n_chunks}")


@pytest.mark.parametrize("cfg_name,T", [("c1", 3000), ("c2", 1337), ("c3", 777)])
def test_baseline_on_bench_shapes(cfg_name, T):
    """The bench's shapes (GQA 4, 3- and 4-bit residuals, strides 8..32) at
    ragged lengths: not a multiple of the 64-key block or of either stride."""
    cfg = dataclasses.replace(synth.CONFIGS[cfg_name], T=T)
    k, v = synth.make_kv(cfg)
    q = synth.make_q(cfg)
    H, D = cfg.n_kv_heads, cfg.head_dim
    ck = O.OracleComponent(H, D, cfg.stride_k, cfg.delta_bits_k, cfg.dead_zone_k, capacity=T)
    cv = O.OracleComponent(H, D, cfg.stride_v, cfg.delta_bits_v, cfg.dead_zone_v, capacity=T)
    ck.append(k[0])
    cv.append(v[0])
    ref, absw = O.sdpa_fused(q[0], ck, cv, D ** -0.5, return_absw=True)
    for n_chunks in (0, 5):
        got = O.fused_decode_f32(q[0], ck, cv, D ** -0.5, n_chunks=n_chunks)
        check(got, ref, absw, f"{cfg_name} T={T} chunks={n_chunks}")


def test_baseline_prefix_and_empty():
    """T below the appended length reads only the first T tokens; T = 0
    gives zeros (the reference kernel's global_sum == 0 branch)."""
    rng = np.random.default_rng(5)
    H, D, T = 2, 64, 200
    x = rng.standard_normal((2, H, T, D)).astype(np.float16)
    ck = O.OracleComponent(H, D, 16, 4, 0.0, capacity=T)
    cv = O.OracleComponent(H, D, 4, 4, 0.0, capacity=T)
    ck.append(x[0])
    cv.append(x[1])
    q = rng.standard_normal((4, D)).astype(np.float16)
    for Tp in (1, 17, 65, 129):
        ref, absw = O.sdpa_fused(q, ck, cv, 0.125, T=Tp, return_absw=True)
        check(O.fused_decode_f32(q, ck, cv, 0.125, T=Tp), ref, absw, f"T={Tp}")
    assert not np.any(O.fused_decode_f32(q, ck, cv, 0.125, T=0))
