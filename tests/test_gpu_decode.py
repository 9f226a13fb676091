"""GPU parity of the fused decode attention against the oracle's restatement of
the reference's reconstruct-fallback path (attention.py:61-74).

Bar (from the BASELINE north star): |got - ref| <= 2e-3 + 1e-2*|ref| elementwise
(and relative L2 <= 1e-2) against the fallback output on identical seeded
inputs; plus a tight bar against the oracle's restatement of the reference's
fused-kernel semantics (kernels.py:79-228), which is what the gfx950 kernels
compute: 2e-4 + 1e-3*|ref| for the portable kernel, 5e-4 + 2e-3*|ref| for the
MFMA kernel, whose P.V operands hold the softmax weights in fp16.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import (assert_close, assert_close_fallback, assert_tight, build_gpu_cache,
                          build_oracle, to_gpu)

pytestmark = pytest.mark.gpu


def decode_gpu(cache, q_np, scale, generic=False, seq_lens=None):
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    q = to_gpu(q_np)
    lens = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    return chronoquant_sdpa_cache_kernel(q, cache, scale, seq_lens=lens, generic=generic).float().cpu().numpy()


def oracle_fallback(ck, cv, q_b, scale):
    return O.sdpa_fallback(q_b[:, None], ck.reconstruct(), cv.reconstruct(), scale)[:, 0]


def run_config(name, T=None, B=None, generic=False, seqs=None, max_abs=None,
               fallback_slack=False):
    """Decode configuration `name` on the GPU and check sequences `seqs`
    (default all) against the oracle; max_abs: also bound max |got - ref|
    against the fallback by that value (the north star's plain max-abs);
    fallback_slack: widen the fallback bar by the fallback's own distance to
    binary64 attention (assert_close_fallback)."""
    from chronoquant_mlx_amd import synth
    cfg = synth.CONFIGS[name]
    B = cfg.B if B is None else B
    k, v = synth.make_kv(cfg, T=T, B=B)
    q = synth.make_q(cfg, B=B)
    params = dict(stride_k=cfg.stride_k, stride_v=cfg.stride_v, bits_k=cfg.delta_bits_k,
                  bits_v=cfg.delta_bits_v, dz_k=cfg.dead_zone_k, dz_v=cfg.dead_zone_v)
    cache = build_gpu_cache(k, v, **params)
    scale = cfg.head_dim ** -0.5
    out = decode_gpu(cache, q, scale, generic=generic)
    for b in (range(B) if seqs is None else seqs):
        ck, cv = build_oracle(k[b], v[b], **params)
        ref = oracle_fallback(ck, cv, q[b], scale)
        if fallback_slack:
            exact = O.sdpa_exact(q[b], ck.reconstruct(), cv.reconstruct(), scale)
            err, _ = assert_close_fallback(out[b], ref, exact, what=f"{name} b={b}")
            assert_close(out[b], exact, what=f"{name} b={b} vs binary64 attention")
        else:
            err, _ = assert_close(out[b], ref, what=f"{name} b={b}")
        if max_abs is not None:
            assert err <= max_abs, f"{name} b={b}: max-abs {err:.3e} > {max_abs}"
        fused, absw = O.sdpa_fused(q[b], ck, cv, scale, return_absw=True)
        if fallback_slack and not generic:
            assert_tight(out[b], fused, what=f"{name} b={b}", absw=absw)
        else:
            assert_tight(out[b], fused, what=f"{name} b={b}", mfma=not generic)


# c0 and c1 outputs stay well inside |o| < 1, so the north star's bar holds
# there as a plain max-abs of 2e-3 as well as in the atol + rtol reading.
@pytest.mark.parametrize("generic", [False, True])
def test_c0_full(generic):
    run_config("c0", generic=generic, max_abs=2e-3)


@pytest.mark.parametrize("generic", [False, True])
def test_c1_full(generic):
    run_config("c1", generic=generic, max_abs=2e-3)


# c2's 8x outlier channels make scores reach +-18, where the fallback's fp16
# score rounding moves single elements by more than the bar; the reference's
# own fused kernel differs from its fallback there too (assert_close_fallback)
def test_c2_two_sequences():
    # Full-Throttle V3, T = 32768: a batch of two (16 splits of 2048 tokens)
    run_config("c2", B=2, fallback_slack=True)


def test_c2_full_batch_plan():
    # configs[2] at its own batch of 8: the plan bench.py times (4 splits of
    # 8192 tokens per (sequence, kv head)); the first and the last sequence
    # are checked against the oracle
    run_config("c2", seqs=(0, 7), fallback_slack=True)


@pytest.mark.parametrize("T", [1, 2, 31, 32, 33, 63, 64, 65, 129, 1000])
def test_short_contexts(T):
    run_config("c1", T=T)


@pytest.mark.parametrize("G,H,D", [(1, 4, 128), (2, 4, 128), (4, 2, 64), (8, 1, 128),
                                   (4, 2, 72), (3, 2, 256), (16, 1, 128)])
def test_shapes(G, H, D):
    rng = np.random.default_rng(G * 100 + D)
    B, T = 2, 700
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=16, stride_v=4)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    for generic in (False, True):
        out = decode_gpu(cache, q, scale, generic=generic)
        for b in range(B):
            ck, cv = build_oracle(k[b], v[b], **params)
            assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"generic={generic}")
            assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"generic={generic}",
                         mfma=not generic)


@pytest.mark.parametrize("sk,sv", [(5, 6), (12, 20), (48, 7), (4, 96), (33, 4)])
def test_strides_not_powers_of_two(sk, sv):
    # the MFMA kernel's float-reciprocal token -> anchor / slot path (power-of
    # two strides take shifts), including strides that do not divide the
    # 64-token chunk and groups that straddle chunks and splits
    rng = np.random.default_rng(sk * 100 + sv)
    B, H, T, D, G = 2, 2, 1500, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=sk, stride_v=sv)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    out = decode_gpu(cache, q, scale)
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b}")
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b}")


@pytest.mark.parametrize("sk,sv", [(4, 8), (8, 4), (16, 32), (32, 128), (128, 16), (64, 64)])
def test_pipelined_plan_strides(sk, sv):
    # Two sequences of 9000 tokens over 8 kv heads: the grid plan gives 9
    # splits of 1024 tokens (two 64-token chunks per wave), so the pipelined
    # instance runs, which loads a chunk's code rows as contiguous slot blocks
    # and scatters them to their tokens.  Strides below, at and above the
    # chunk, and a last split that ends inside a chunk (waves past the end).
    rng = np.random.default_rng(sk * 1000 + sv)
    B, H, T, D, G = 2, 8, 9000, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=sk, stride_v=sv)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    out = decode_gpu(cache, q, scale)
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b}")
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b}")


@pytest.mark.parametrize("sk,sv", [(4, 8), (8, 4), (16, 32), (64, 32), (128, 16), (64, 64)])
def test_balanced_plan_strides(sk, sv):
    # Ragged lengths over 8 kv heads take the balanced partition, whose
    # instance also loads a chunk's code rows as contiguous slot blocks and
    # scatters them to their tokens: strides below, at and above the chunk,
    # segments that start inside a sequence at a 512-token unit boundary,
    # and sequences that end inside a chunk.
    rng = np.random.default_rng(sk * 1000 + sv + 7)
    B, H, T, D, G = 12, 8, 3000, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    lens = rng.integers(1, T + 1, size=B)
    lens[:4] = [T, 1, 513, 2049]
    params = dict(stride_k=sk, stride_v=sv)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    out = decode_gpu(cache, q, scale, seq_lens=lens.tolist())
    for b, L in enumerate(lens.tolist()):
        ck, cv = build_oracle(k[b, :, :L], v[b, :, :L], **params)
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b} L={L}")
        if b < 3:
            assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b} L={L}")


def test_pipelined_plan_single_split():
    # 40 sequences x 8 kv heads fill the grid without splitting: one
    # workgroup per (sequence, kv head) over 640 tokens, so the pipelined
    # instance runs with two chunks on waves 0-1 and one on the others, and
    # writes the output without a fold.
    rng = np.random.default_rng(77)
    B, H, T, D, G = 40, 8, 640, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=64, stride_v=32)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    out = decode_gpu(cache, q, scale)
    for b in (0, 17, 39):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b}")
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b}")


def test_workspace_shared_across_shapes():
    # regression: calls with different split counts share the per-device
    # workspace; counters must stay valid between them
    rng = np.random.default_rng(31)
    H, D, G = 8, 128, 4
    params = dict(stride_k=32, stride_v=8)
    runs = []
    for B, T in ((1, 5000), (2, 65), (1, 16384), (3, 700), (1, 65), (2, 129)):
        k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
        v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
        q = rng.standard_normal((B, G * H, D)).astype(np.float16)
        runs.append((build_gpu_cache(k, v, **params), k, v, q))
    for _ in range(2):
        for cache, k, v, q in runs:
            out = decode_gpu(cache, q, D ** -0.5)
            for b in range(k.shape[0]):
                ck, cv = build_oracle(k[b], v[b], **params)
                assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, D ** -0.5), what=f"T={k.shape[2]}")


@pytest.mark.parametrize("generic", [False, True])
@pytest.mark.parametrize("lens", [[2000, 1, 1057, 640], [0, 2000, 513, 512], [511, 1, 2000, 0]])
def test_ragged_lengths(generic, lens):
    # per-sequence lengths: sequence b reads only its first L_b tokens and
    # must equal an independent cache of length L_b.  The split plan follows
    # the longest length (4 splits of 512 here), so shorter sequences leave
    # later splits empty: those workgroups exit and the combine counts only
    # the live ones.  An empty sequence answers zeros.
    rng = np.random.default_rng(21)
    B, H, T, D, G = 4, 8, 2000, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    # twice: the second call reuses the workspace and counters of the first
    for _ in range(2):
        out = decode_gpu(cache, q, scale, seq_lens=lens, generic=generic)
        for b, L in enumerate(lens):
            if L == 0:
                assert np.array_equal(out[b], np.zeros_like(out[b])), f"b={b} L=0"
                continue
            ck, cv = build_oracle(k[b, :, :L], v[b, :, :L], **params)
            assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b} L={L}")
            assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b} L={L}",
                         mfma=not generic)


@pytest.mark.parametrize("B,H,T,G,sk,sv,seed", [
    (40, 8, 3000, 4, 32, 8, 41), (1030, 1, 96, 4, 32, 8, 42),
    (40, 2, 3000, 8, 32, 8, 44), (24, 2, 2600, 20, 12, 20, 45), (1030, 1, 96, 8, 16, 4, 46)])
def test_balanced_plan_many_sequences(B, H, T, G, sk, sv, seed):
    # The MFMA kernels lay the batch's 512-token units end to end and give
    # every workgroup of a (kv head, q-head chunk) column the same share, so
    # a workgroup's range ends one sequence and starts the next, and a
    # sequence's pieces combine across workgroups.  B=40 / 24 use the
    # per-sequence unit table (lengths 0..T); B=1030 is past the table's 1024
    # sequences and takes the uniform unit space, where each workgroup covers
    # several sequences.  G=4 with power-of-two strides runs the GQA-4
    # kernel; G=8 and G=20 (two q-head chunks, strides 12 / 20 on the
    # float-reciprocal path) the 16-head kernel.
    rng = np.random.default_rng(seed)
    D = 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    lens = rng.integers(0, T + 1, size=B)
    lens[:3] = [0, T, 1]
    params = dict(stride_k=sk, stride_v=sv)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    for _ in range(2):
        out = decode_gpu(cache, q, scale, seq_lens=lens.tolist())
        for b, L in enumerate(lens.tolist()):
            if L == 0:
                assert np.array_equal(out[b], np.zeros_like(out[b])), f"b={b} L=0"
                continue
            ck, cv = build_oracle(k[b, :, :L], v[b, :, :L], **params)
            assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b} L={L}")
            if b < 8:
                assert_close(out[b], oracle_fallback(ck, cv, q[b], scale), what=f"b={b} L={L}")


@pytest.mark.parametrize("G", [4, 8])
def test_uniform_batch_ranges_across_sequences(G):
    # 3 sequences of 16384 tokens over 32 workgroups per column: 3 units per
    # workgroup, so some workgroups end one sequence and start the next.
    rng = np.random.default_rng(43)
    B, H, T, D = 3, 8, 16384, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.05, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.05, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    out = decode_gpu(cache, q, scale)
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        assert_tight(out[b], O.sdpa_fused(q[b], ck, cv, scale), what=f"b={b}")


def test_output_dtypes_and_fp32_queries():
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    rng = np.random.default_rng(5)
    B, H, T, D = 1, 2, 300, 128
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, 4 * H, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8)
    cache = build_gpu_cache(k, v, **params)
    ck, cv = build_oracle(k[0], v[0], **params)
    fused = O.sdpa_fused(q[0], ck, cv, 0.3)
    out16 = decode_gpu(cache, q, 0.3)
    assert_tight(out16[0], fused)
    # fp32 output: no output rounding; what remains is the fp16 rounding of the
    # softmax weights fed to the MFMA P.V (<= 2^-12 relative per weight, the
    # rounding point the reference fallback also has) and fp32 accumulation
    out32 = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, 0.3, out_dtype=torch.float32)
    assert_close(out32[0].cpu().numpy(), fused, 5e-5, 2.5e-4)
    out32g = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, 0.3, out_dtype=torch.float32, generic=True)
    assert_close(out32g[0].cpu().numpy(), fused, 2e-5, 1e-5)  # portable kernel: fp32 weights
    # fp32 queries: q*scale is not rounded to fp16; compare with binary64
    # attention on the reconstruction
    outq = chronoquant_sdpa_cache_kernel(to_gpu(q, torch.float32), cache, 0.3).cpu().numpy()
    exact = O.sdpa_exact(q[0], ck.reconstruct(), cv.reconstruct(), 0.3)
    assert_close(outq[0], exact)


@pytest.mark.parametrize("out_dtype", ["f16", "bf16", "f32"])
def test_split_fold_outputs_and_short_bound_lengths(out_dtype):
    # The split fold of the grid plan (several splits of one sequence fold
    # their partials into the output) with every output dtype, and with a
    # device length shorter than the cache, so that fewer splits than the
    # plan's hold tokens: T=3000 gives 6 splits of 512 tokens, length 1300
    # leaves 3 of them live.
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[out_dtype]
    rng = np.random.default_rng(31 + len(out_dtype))
    B, H, T, D, G = 1, 8, 3000, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    params = dict(stride_k=32, stride_v=8)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    # bf16 output: one more rounding of |o| < 1 at 2^-9 relative
    atol, rtol = {"f16": (5e-4, 2e-3), "bf16": (2e-3, 8e-3), "f32": (5e-5, 2.5e-4)}[out_dtype]
    for L in (T, 1300):
        lens = None if L == T else torch.tensor([L], dtype=torch.int32, device="cuda")
        out = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, scale, out_dtype=dt,
                                      seq_lens=lens).float().cpu().numpy()
        ck, cv = build_oracle(k[0][:, :L], v[0][:, :L], **params)
        assert_close(out[0], oracle_fallback(ck, cv, q[0], scale), what=f"{out_dtype} L={L}")
        assert_close(out[0], O.sdpa_fused(q[0], ck, cv, scale), atol, rtol,
                     what=f"{out_dtype} L={L} vs fused semantics")


@pytest.mark.parametrize("B,H,G,T,lens", [
    (2, 8, 4, 3000, None),
    (1, 8, 4, 16384, None),          # configs[1]'s shape, the one bench.py times
    (3, 2, 2, 777, [1, 500, 777]),   # per-sequence lengths, a one-token sequence
    (1, 1, 4, 65536, None),          # 128 splits: split-ready flags instead of records
    (2, 4, 1, 1000, None),
    (1, 2, 8, 700, None),            # GQA 8: the stride-1 compressed-cache kernels
])
def test_fp16_baseline_matches_exact(B, H, G, T, lens):
    # cq_fp16_decode_attn (the uncompressed flash decode the compressed path is
    # compared with) against binary64 attention on the same fp16 K/V
    from chronoquant_mlx_amd import _lib, synth
    D = 128
    if (B, H, G, T) == (1, 8, 4, 16384):
        k, v = synth.make_kv(synth.CONFIGS["c1"])
        q = synth.make_q(synth.CONFIGS["c1"])
    else:
        rng = np.random.default_rng(8 + T)
        k = rng.standard_normal((B, H, T, D)).astype(np.float16)
        v = rng.standard_normal((B, H, T, D)).astype(np.float16)
        q = rng.standard_normal((B, G * H, D)).astype(np.float16)
    kt, vt, qt = to_gpu(k), to_gpu(v), to_gpu(q)
    out = torch.full((B, G * H, D), float("nan"), dtype=torch.float16, device="cuda")
    need = _lib.load().cq_decode_workspace_size(B, H, G * H, D, T)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    lt = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    _lib.call("cq_fp16_decode_attn", kt.data_ptr(), vt.data_ptr(), T, B, H, D, qt.data_ptr(),
              _lib.CQ_F16, G * H, float(D ** -0.5), _lib.ptr(lt), T, T, out.data_ptr(),
              _lib.CQ_F16, ws.data_ptr(), need, _lib.stream_of(qt))
    got = out.float().cpu().numpy()
    for b in range(B):
        L = T if lens is None else lens[b]
        ref = O.sdpa_exact(q[b], k[b][:, :L], v[b][:, :L], D ** -0.5)
        assert_close(got[b], ref, what=f"fp16 baseline b={b}")
        assert_tight(got[b], ref, what=f"fp16 baseline b={b} (binary64)")


def test_sdpa_dispatch_and_fallback():
    # q_len > 1 takes the reconstruct fallback with the "causal" mask
    from chronoquant_mlx_amd import chronoquant_sdpa
    rng = np.random.default_rng(6)
    B, H, T, D, G, Tq = 1, 2, 200, 64, 2, 7
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((B, G * H, Tq, D)).astype(np.float16)
    params = dict(stride_k=8, stride_v=4)
    cache = build_gpu_cache(k, v, **params)
    out = chronoquant_sdpa(to_gpu(q), None, None, cache, D ** -0.5, mask="causal")
    ck, cv = build_oracle(k[0], v[0], **params)
    ref = O.sdpa_fallback(q[0], ck.reconstruct(), cv.reconstruct(), D ** -0.5, causal=True)
    assert_close(out[0].float().cpu().numpy(), ref.astype(np.float32))
    # single query: fused path == fallback path within the bar
    out1 = chronoquant_sdpa(to_gpu(q[:, :, -1:]), None, None, cache, D ** -0.5)
    cache.use_fused = False
    out2 = chronoquant_sdpa(to_gpu(q[:, :, -1:]), None, None, cache, D ** -0.5)
    assert_close(out1.float().cpu().numpy(), out2.float().cpu().numpy())


def test_patch_routes_chronoquant_caches():
    import chronoquant_mlx_amd as cq
    from chronoquant_mlx_amd import host
    rng = np.random.default_rng(3)
    k = to_gpu(rng.standard_normal((1, 2, 40, 64)).astype(np.float16))
    q = to_gpu(rng.standard_normal((1, 4, 1, 64)).astype(np.float16))
    plain = host.KVCache()
    kk, vv = plain.update_and_fetch(k, k)
    ref = host.scaled_dot_product_attention(q, kk, vv, plain, 0.125, None)
    cq.apply()
    try:
        c = cq.ChronoQuantCache(stride_k=1, stride_v=1)
        c.update_and_fetch(k, k)
        got = host.scaled_dot_product_attention(q, k, k, c, 0.125, None)
        # stride 1: every token is an exact fp16 I-frame -> same attention
        assert_close(got.float().cpu().numpy(), ref.float().cpu().numpy())
        again = host.scaled_dot_product_attention(q, kk, vv, plain, 0.125, None)
        assert torch.equal(again, ref)
    finally:
        cq.revert()
    assert host.scaled_dot_product_attention is not None


def test_bf16_queries():
    # bf16 queries: q' = bf16(q * bf16(scale)) (attention.py:46 in bf16), fed to
    # the MFMA kernel as fp16 (exact in fp16's normal range) and to the
    # portable kernel as fp32; both against binary64 attention on the fp16
    # reconstruction with the same q'
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    rng = np.random.default_rng(17)
    B, H, T, D, G = 2, 2, 900, 128, 4
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q32 = rng.standard_normal((B, G * H, D)).astype(np.float32)
    params = dict(stride_k=32, stride_v=8)
    cache = build_gpu_cache(k, v, **params)
    scale = D ** -0.5
    qb = torch.from_numpy(q32).to("cuda").to(torch.bfloat16)
    out_m = chronoquant_sdpa_cache_kernel(qb, cache, scale).float().cpu().numpy()
    out_g = chronoquant_sdpa_cache_kernel(qb, cache, scale, generic=True).float().cpu().numpy()
    scb = torch.tensor(scale, dtype=torch.bfloat16)
    qprime = (qb.cpu() * scb).to(torch.float16).numpy()  # bf16 product, exactly representable
    for b in range(B):
        ck, cv = build_oracle(k[b], v[b], **params)
        exact = O.sdpa_exact(qprime[b], ck.reconstruct(), cv.reconstruct(), 1.0)
        # bf16 output rounding: 2^-9 relative
        assert_close(out_m[b], exact, 2e-3, 1e-2, what=f"mfma b={b}")
        assert_close(out_g[b], exact, 2e-3, 1e-2, what=f"generic b={b}")
        assert_close(out_m[b], out_g[b], 5e-4, 5e-3, what=f"mfma vs generic b={b}")
