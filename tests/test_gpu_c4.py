"""configs[4] against the oracle: the chunked-prefill kernel at the exact shape
bench.py times, and the full-size Qwen-style decoder's layer caches and
attention outputs.

Reference: the end-to-end runs fill every cache slot of the model with
create_full_throttle_caches (patch.py:91-104) and route its attention through
chronoquant_sdpa: q_len > 1 takes the reconstruct fallback
(attention.py:61-74 over cache.py:131-160), q_len == 1 the fused decode
(attention.py:45-59).  Keys are cached after RoPE (mlx_lm's order).  The
model's K/V are bf16, so the codec runs in bf16 arithmetic with fp16
I-frames (cache.py:104, :113).

Bar: codes, packed words, scales and I-frames bit for bit; attention within
|d| <= 2e-3 + 1e-2 |ref| and relative L2 <= 1e-2 of the oracle fallback.
With bf16 queries the reference's fallback computes bf16 x fp16 in fp32
(MLX's promotion: fp32 scores and weights, one rounding to bf16), which the
oracle restates as sdpa_fallback_bf16q.
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import assert_close, build_gpu_cache, build_oracle, to_gpu

pytestmark = pytest.mark.gpu

FTV3 = dict(stride_k=64, stride_v=32, bits_k=4, bits_v=3, dz_k=0.0, dz_v=0.05)


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _bf16_fallback(q_bf16: torch.Tensor, rk, rv, scale: float, causal: bool) -> np.ndarray:
    """Oracle fallback for bf16 queries q [nq, Lq, D] -> float64 [nq, Lq, D]."""
    out = O.sdpa_fallback_bf16q(_bf16_bits(q_bf16), np.ascontiguousarray(rk),
                                np.ascontiguousarray(rv), scale, causal=causal)
    return O.bf16_to_f32(out).astype(np.float64)


@pytest.mark.parametrize("qdtype", ["f16", "bf16"])
def test_prefill_c4_chunk_shape(qdtype):
    # the last 512-token chunk of an 8192-token prompt, GQA 32/8, FT-V3:
    # exactly the call bench.py's prefill line times (same split plan)
    from chronoquant_mlx_amd import synth
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel
    T, L, D = 8192, 512, 128
    cfg = dataclasses.replace(synth.CONFIGS["ftv3_16k"], T=T)
    k, v = synth.make_kv(cfg)
    print(f"prefill c4 chunk: T={T} L={L} q {qdtype}", flush=True)
    cache = build_gpu_cache(k, v, **FTV3)
    rng = np.random.default_rng(8192)
    q32 = rng.standard_normal((1, cfg.n_q_heads, L, D)).astype(np.float32)
    scale = D ** -0.5
    ck, cv = build_oracle(k[0], v[0], **FTV3)
    rk, rv = ck.reconstruct(), cv.reconstruct()
    if qdtype == "f16":
        q = to_gpu(q32.astype(np.float16))
        ref = O.sdpa_fallback(q32[0].astype(np.float16), rk, rv, scale,
                              causal=True).astype(np.float64)
    else:
        q = torch.from_numpy(q32).to("cuda").to(torch.bfloat16)
        ref = _bf16_fallback(q[0], rk, rv, scale, causal=True)
    out = chronoquant_prefill_kernel(q, cache, scale, causal=True)
    assert out.dtype == q.dtype
    err, rel = assert_close(out.float().cpu().numpy()[0], ref, what=f"c4 chunk {qdtype}")
    print(f"prefill c4 chunk {qdtype}: max-abs {err:.2e} rel {rel:.2e}", flush=True)


class _Recorder:
    """Records, for one layer's cache, the post-RoPE K/V it is given (prefill
    chunks through update_and_fetch; decode tokens through the fused
    norm + RoPE + append, whose K/V are recomputed by the two-step path it
    is bit-identical to) and the q / attention output of each call."""

    def __init__(self, cache, n_kv):
        from chronoquant_mlx_amd.models import fused
        self.k, self.v, self.q, self.o = [], [], [], []
        up, fa = cache.update_and_fetch, cache.fused_decode_append

        def update_and_fetch(keys, values):
            self.k.append(keys.detach().clone())
            self.v.append(values.detach().clone())
            return up(keys, values)

        def fused_decode_append(qkv, n_q_heads, q_weight, k_weight, cos, sin, positions, eps):
            q2, k2, v2 = fused.qkv_norm_rope(qkv, n_q_heads, n_kv, q_weight, k_weight, cos, sin,
                                             positions.reshape(-1), eps)
            q = fa(qkv, n_q_heads, q_weight, k_weight, cos, sin, positions, eps)
            assert q is not None and torch.equal(q.view(torch.int16), q2.view(torch.int16))
            self.k.append(k2)
            self.v.append(v2)
            return q

        cache.update_and_fetch = update_and_fetch
        cache.fused_decode_append = fused_decode_append


def test_c4_model_layers_against_oracle():
    from chronoquant_mlx_amd import create_full_throttle_caches, patch, synth
    from chronoquant_mlx_amd.models import qwen
    args = qwen.ModelArgs()  # configs[4]: 32 layers, hidden 4096, GQA 32/8, SwiGLU 12288
    prompt_len, chunk, n_dec = 8192, 512, 12
    H, D, nq = args.num_key_value_heads, args.head_dim, args.num_attention_heads
    print("c4 model: building the full-size random model", flush=True)
    model = qwen.random_model(args, seed=0)
    prompt = torch.randint(0, args.vocab_size, (1, prompt_len),
                           generator=torch.Generator().manual_seed(0)).cuda()
    layers = (0, args.num_hidden_layers - 1)
    patch.apply()
    try:
        caches = create_full_throttle_caches(model)
        recs = {i: _Recorder(caches[i], H) for i in layers}
        by_cache = {id(caches[i]): recs[i] for i in layers}
        patched = qwen.scaled_dot_product_attention

        def sdpa(queries, keys, values, cache, scale, mask=None, **kw):
            out = patched(queries, keys, values, cache=cache, scale=scale, mask=mask, **kw)
            r = by_cache.get(id(cache))
            if r is not None:
                r.q.append(queries.detach().clone())
                r.o.append(out.detach().clone())
            return out

        qwen.scaled_dot_product_attention = sdpa
        toks, _, _ = qwen.generate(model, caches, prompt, n_dec + 1, prefill_chunk=chunk,
                                   graph=False)
    finally:
        patch.revert()
    torch.cuda.synchronize()
    T = prompt_len + n_dec
    print(f"c4 model: prefill + {n_dec} decode steps done", flush=True)

    # KV bytes: every layer holds the reference's nbytes for T tokens
    per_layer = synth.compressed_bytes(T, H, D, 64, 32)
    assert all(c.offset == T for c in caches)
    assert sum(c.nbytes for c in caches) == args.num_hidden_layers * per_layer

    scale = D ** -0.5
    for i in layers:
        r = recs[i]
        assert len(r.k) == prompt_len // chunk + n_dec and len(r.o) == len(r.k)
        k_all = _bf16_bits(torch.cat(r.k, dim=2))[0]  # [H, T, D] bf16 bits
        v_all = _bf16_bits(torch.cat(r.v, dim=2))[0]
        ck = O.OracleComponent(H, D, 64, 4, 0.0, capacity=T)
        cv = O.OracleComponent(H, D, 32, 3, 0.05, capacity=T)
        ck.append(k_all, "bf16")
        cv.append(v_all, "bf16")
        st = caches[i].state
        for j, comp in ((0, ck), (1, cv)):
            kf, pk, sc = comp.active()
            assert np.array_equal(st[j][0].cpu().numpy().view(np.uint16), kf.view(np.uint16)), \
                f"layer {i} keyframes[{j}]"
            assert np.array_equal(st[2 + 2 * j][0].cpu().numpy(), pk), f"layer {i} packed[{j}]"
            assert np.array_equal(st[3 + 2 * j][0].cpu().numpy().view(np.uint16),
                                  sc.view(np.uint16)), f"layer {i} scales[{j}]"
        rk, rv = ck.reconstruct(), cv.reconstruct()
        # the first and the last prefill chunk (MFMA prefill kernel), and every
        # decode step (fused decode kernel), each over the cache as it was then
        n_pre = prompt_len // chunk
        for c in (0, n_pre - 1) + tuple(range(n_pre, n_pre + n_dec)):
            Tc = (c + 1) * chunk if c < n_pre else prompt_len + (c - n_pre) + 1
            q = r.q[c][0]  # [nq, Lq, D] bf16, unscaled
            ref = _bf16_fallback(q, rk[:, :Tc], rv[:, :Tc], scale, causal=q.shape[1] > 1)
            got = r.o[c].float().cpu().numpy()[0]
            assert got.shape == (nq, q.shape[1], D)
            err, rel = assert_close(got, ref, what=f"layer {i} call {c} T={Tc}")
            print(f"c4 model: layer {i} call {c} (T={Tc}) max-abs {err:.2e} rel {rel:.2e}",
                  flush=True)

    # ---- the same generation with the decode steps replayed from one HIP
    # graph (the form bench.py times): the captured step records its layer
    # 0 / 31 queries and outputs into device buffers at the step index
    # position - prompt_len, so each replay's are kept
    patch.apply()
    try:
        caches_g = create_full_throttle_caches(model)
        slot = {id(caches_g[i]): i for i in layers}
        qb = {i: torch.zeros(n_dec, 1, nq, 1, D, dtype=torch.bfloat16, device="cuda")
              for i in layers}
        ob = {i: torch.zeros_like(qb[i]) for i in layers}

        def sdpa_g(queries, keys, values, cache, scale, mask=None, **kw):
            out = patched(queries, keys, values, cache=cache, scale=scale, mask=mask, **kw)
            i = slot.get(id(cache))
            if i is not None and cache._dev_pos is not None:  # a decode step
                idx = (cache._dev_pos[:1].long() - prompt_len).clamp(0, n_dec - 1)
                qb[i].index_copy_(0, idx, queries.detach()[None])
                ob[i].index_copy_(0, idx, out.detach()[None])
            return out

        qwen.scaled_dot_product_attention = sdpa_g
        toks_g, _, _ = qwen.generate(model, caches_g, prompt, n_dec + 1, prefill_chunk=chunk,
                                     graph=True)
    finally:
        patch.revert()
    torch.cuda.synchronize()
    print(f"c4 model: graph-captured decode of {n_dec} steps done", flush=True)
    assert torch.equal(toks_g, toks), "graph decode chose other tokens than eager decode"
    # every layer's cache after the graph replays equals the eager run's
    for li, (cg, ce) in enumerate(zip(caches_g, caches)):
        assert cg.offset == ce.offset == T
        for x, y in zip(cg.state, ce.state):
            assert torch.equal(x.view(torch.int16) if x.dtype != torch.uint32 else x,
                               y.view(torch.int16) if y.dtype != torch.uint32 else y), \
                f"layer {li}: graph-decoded cache state differs"
    for i in layers:
        r = recs[i]  # the eager run's K/V: the same bits (states are equal)
        ck = O.OracleComponent(H, D, 64, 4, 0.0, capacity=T)
        cv = O.OracleComponent(H, D, 32, 3, 0.05, capacity=T)
        ck.append(_bf16_bits(torch.cat(r.k, dim=2))[0], "bf16")
        cv.append(_bf16_bits(torch.cat(r.v, dim=2))[0], "bf16")
        rk, rv = ck.reconstruct(), cv.reconstruct()
        for sidx in range(n_dec):
            Tc = prompt_len + sidx + 1
            q = qb[i][sidx, 0, :]  # [nq, 1, D]
            assert torch.equal(q.view(torch.int16), r.q[n_pre + sidx][0].view(torch.int16)), \
                f"layer {i} graph step {sidx}: query differs from the eager step's"
            ref = _bf16_fallback(q, rk[:, :Tc], rv[:, :Tc], scale, causal=False)
            got = ob[i][sidx, 0].float().cpu().numpy()
            err, rel = assert_close(got, ref, what=f"layer {i} graph step {sidx} T={Tc}")
        print(f"c4 model: layer {i} graph steps vs oracle ok (last max-abs {err:.2e})", flush=True)
