"""The fused decode operator called with the reference's signature
(kernels.py:248-279), exactly as the reference's attention.py:46-58 calls it,
and the host-observable split-wait status (cq_decode_status)."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import assert_close, assert_tight, build_gpu_cache, build_oracle, to_gpu

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def reference_style_call(cache, queries, scale):
    """attention.py:46-58 of the reference, with this library's operator."""
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_kernel
    batch, n_q_heads, q_len, head_dim = queries.shape
    # fp16 queries * weak scalar scale -> fp16, then fp32 (attention.py:46)
    q = (queries * torch.tensor(scale, dtype=queries.dtype, device=queries.device)).reshape(
        n_q_heads, head_dim).to(torch.float32)
    out = chronoquant_sdpa_kernel(
        q=q,
        keyframes_k=cache.kernel_keyframes_k(),
        packed_k=cache.kernel_packed_k(),
        scales_k=cache.kernel_scales_k(),
        keyframes_v=cache.kernel_keyframes_v(),
        packed_v=cache.kernel_packed_v(),
        scales_v=cache.kernel_scales_v(),
        seq_len=cache.offset,
        stride_k=cache.stride_k,
        stride_v=cache.stride_v,
    )
    assert out.dtype == torch.float32 and out.shape == (n_q_heads, head_dim)
    return out.reshape(batch, n_q_heads, q_len, head_dim).to(queries.dtype), out


@pytest.mark.parametrize("name", ["c1", "ftv3_16k"])
def test_reference_signature_at_full_size(name):
    from chronoquant_mlx_amd import synth
    cfg = synth.CONFIGS[name]
    k, v = synth.make_kv(cfg)
    q = synth.make_q(cfg)
    params = dict(stride_k=cfg.stride_k, stride_v=cfg.stride_v, bits_k=cfg.delta_bits_k,
                  bits_v=cfg.delta_bits_v, dz_k=cfg.dead_zone_k, dz_v=cfg.dead_zone_v)
    cache = build_gpu_cache(k, v, **params)
    scale = cfg.head_dim ** -0.5
    print(f"[op] {name}: T={cfg.T}", flush=True)
    out16, out32 = reference_style_call(cache, to_gpu(q[0])[None, :, None, :], scale)
    got = out32.cpu().numpy()
    ck, cv = build_oracle(k[0], v[0], **params)
    fused = O.sdpa_fused(q[0], ck, cv, scale)
    assert_tight(got, fused, what=f"{name} reference-signature operator")
    fb = O.sdpa_fallback(q[0][:, None], ck.reconstruct(), cv.reconstruct(), scale)[:, 0]
    err, _ = assert_close(out16[0, :, 0].float().cpu().numpy(), fb, what=f"{name} vs fallback")
    if name == "c1":  # outputs well inside |o| < 1: the plain max-abs reading holds too
        assert err <= 2e-3
    # the same numbers as the cache-object form of the operator
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    alt = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, scale, out_dtype=torch.float32)
    assert torch.equal(alt[0], out32)


@pytest.mark.parametrize("T,sk,sv", [(1, 32, 8), (2, 32, 8), (40, 1, 8), (300, 16, 1), (777, 32, 8)])
def test_reference_signature_edges(T, sk, sv):
    # placeholders (no P-frames yet, stride 1 components) and short contexts
    rng = np.random.default_rng(T + sk)
    H, G, D = 8, 4, 128
    k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((1, G * H, D)).astype(np.float16)
    cache = build_gpu_cache(k, v, stride_k=sk, stride_v=sv)
    scale = D ** -0.5
    _, out32 = reference_style_call(cache, to_gpu(q)[:, :, None, :], scale)
    ck, cv = build_oracle(k[0], v[0], stride_k=sk, stride_v=sv)
    fused = O.sdpa_fused(q[0], ck, cv, scale)
    assert_tight(out32.cpu().numpy(), fused, what=f"T={T} strides {sk}/{sv}")


def test_reference_signature_contiguous_copies_and_fp32_q():
    # operands handed over as standalone contiguous tensors (not views of a
    # cache), and a q that is not fp16-representable (portable kernel)
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_kernel
    rng = np.random.default_rng(7)
    H, G, D, T = 4, 4, 128, 1500
    k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((1, G * H, D)).astype(np.float16)
    cache = build_gpu_cache(k, v, stride_k=32, stride_v=8)
    scale = D ** -0.5
    ops = [t.contiguous().clone() for t in (
        cache.kernel_keyframes_k(), cache.kernel_packed_k(), cache.kernel_scales_k(),
        cache.kernel_keyframes_v(), cache.kernel_packed_v(), cache.kernel_scales_v())]
    ops[1] = ops[1].view(torch.int32)  # an int32 view of the words is accepted too
    q32 = (to_gpu(q[0]) * torch.tensor(scale, dtype=torch.float16, device="cuda")).float()
    a = chronoquant_sdpa_kernel(q32, *ops, seq_len=T, stride_k=32, stride_v=8)
    _, b = reference_style_call(cache, to_gpu(q)[:, :, None, :], scale)
    assert torch.equal(a, b)
    ck, cv = build_oracle(k[0], v[0], stride_k=32, stride_v=8)
    fused = O.sdpa_fused(q[0], ck, cv, scale)
    qp = q32 * (1 + 1e-6)  # off the fp16 grid: the portable kernel on fp32 q
    c = chronoquant_sdpa_kernel(qp, *ops, seq_len=T, stride_k=32, stride_v=8)
    assert_tight(c.cpu().numpy(), fused, what="fp32 q", mfma=False)
    with pytest.raises(ValueError):
        chronoquant_sdpa_kernel(q32, *ops, seq_len=T + 500, stride_k=32, stride_v=8)


def _decode_into(L, cache, q, out, ws, scale):
    from chronoquant_mlx_amd import _lib
    st = L.cq_decode_attn(cache._descriptor(), q.data_ptr(), _lib.CQ_F16, q.shape[1], scale, None,
                          cache.offset, cache.offset, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(),
                          ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.status_string(st)


@pytest.mark.parametrize("H,G,T", [(8, 4, 16384),   # fold records (32 splits per kv head)
                                   (1, 4, 65536)])  # split-ready flags (128 splits)
def test_forced_poll_timeout_is_reported_then_cleared(H, G, T):
    # A split wait forced to give up after one poll round (the host-side test
    # hook; every kernel still exits normally): the decode must either be
    # right or report CQ_ERR_TIMEOUT, and after the report the workspace is
    # clean, so the next call is bit-identical to a normal one.
    from chronoquant_mlx_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(H * T)
    D = 128
    k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.05, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.05, axis=2).astype(np.float16)
    cache = build_gpu_cache(k, v, stride_k=32, stride_v=8)
    q = to_gpu(rng.standard_normal((1, G * H, D)))
    need = L.cq_decode_workspace_size(1, H, G * H, D, T)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.empty(1, G * H, D, dtype=torch.float16, device="cuda")
    _decode_into(L, cache, q, ref, ws, D ** -0.5)
    assert L.cq_decode_status(ws.data_ptr(), stream) == 0
    out = torch.full_like(ref, float("nan"))
    prev = L.cq_set_fold_poll_bound(1)
    try:
        assert prev == 1 << 20
        _decode_into(L, cache, q, out, ws, D ** -0.5)
        st = L.cq_decode_status(ws.data_ptr(), stream)
    finally:
        L.cq_set_fold_poll_bound(0)
    print(f"[op] H={H} T={T}: status after a one-round poll bound = {st}", flush=True)
    assert st in (0, _lib.CQ_ERR_TIMEOUT)
    if st == 0:  # nothing ran out: then the result is the normal one
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert L.cq_decode_status(ws.data_ptr(), stream) == 0  # cleared by the query
    for _ in range(2):
        again = torch.full_like(ref, float("nan"))
        _decode_into(L, cache, q, again, ws, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
    assert L.cq_decode_status(ws.data_ptr(), stream) == 0


def test_status_query_of_the_noalloc_scratch():
    from chronoquant_mlx_amd import _lib
    L = _lib.load()
    assert L.cq_decode_status(None, torch.cuda.current_stream().cuda_stream) == 0


def test_two_graphs_on_torchs_default_capture_stream():
    # Two graphs captured with torch.cuda.graph(g) (torch's one class-level
    # capture stream) each get their own split workspace: replaying the
    # second before the first, and eager calls in between, all equal eager.
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
    rng = np.random.default_rng(3)
    H, G, D = 8, 4, 128
    caches, qs, refs = [], [], []
    for i, T in enumerate((5000, 9000)):
        k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
        v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
        caches.append(build_gpu_cache(k, v, stride_k=32, stride_v=8))
        qs.append(to_gpu(rng.standard_normal((1, G * H, D))))
        refs.append(chronoquant_sdpa_cache_kernel(qs[i], caches[i], D ** -0.5).clone())
    graphs, outs = [], []
    for i in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(chronoquant_sdpa_cache_kernel(qs[i], caches[i], D ** -0.5))
        graphs.append(g)
    for order in ((1, 0), (0, 1), (1, 1, 0)):
        for i in order:
            outs[i].fill_(float("nan"))
            graphs[i].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[i].view(torch.int16), refs[i].view(torch.int16)), (order, i)
            e = chronoquant_sdpa_cache_kernel(qs[1 - i], caches[1 - i], D ** -0.5)
            assert torch.equal(e.view(torch.int16), refs[1 - i].view(torch.int16))


def test_split_length_knob_other_kernels():
    # CQ_DECODE_SPLIT_TOKENS (the bench's split sweep knob, whole 512-token
    # granules only) over the 16-head and the portable kernels, in a process
    # of its own since the library reads it once
    script = r'''
import numpy as np, sys, torch
sys.path.insert(0, sys.argv[1])
from oracle import oracle as O
from tests.cqtest import build_gpu_cache, build_oracle, to_gpu, assert_tight
from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel
rng = np.random.default_rng(5)
for G, H, sk, sv, generic in ((8, 2, 32, 8, False), (4, 2, 48, 24, False), (4, 2, 32, 8, True)):
    T, D = 5000, 128
    k = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((1, H, T, D)) * 0.1, axis=2).astype(np.float16)
    q = rng.standard_normal((1, G * H, D)).astype(np.float16)
    cache = build_gpu_cache(k, v, stride_k=sk, stride_v=sv)
    out = chronoquant_sdpa_cache_kernel(to_gpu(q), cache, D ** -0.5, generic=generic)
    ck, cv = build_oracle(k[0], v[0], stride_k=sk, stride_v=sv)
    assert_tight(out[0].float().cpu().numpy(), O.sdpa_fused(q[0], ck, cv, D ** -0.5),
                 what=f"G={G} strides {sk}/{sv} generic={generic}", mfma=not generic)
print("knob ok", flush=True)
'''
    env = dict(os.environ, CQ_DECODE_SPLIT_TOKENS="1024")
    r = subprocess.run([sys.executable, "-c", script, ROOT], env=env, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "knob ok" in r.stdout
