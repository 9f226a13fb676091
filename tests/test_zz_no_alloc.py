"""cq_decode_attn_noalloc, the decode entry point that allocates nothing (its
split partials and counters live in a static per-GPU device array), against
cq_decode_attn with a caller workspace: same kernels and plan, so the outputs
must be bit-identical.  No counterpart in the reference; this entry point is
for callers that cannot allocate (HIP graph capture, serving loops)."""
import numpy as np
import pytest
import torch

from tests.cqtest import build_gpu_cache, to_gpu

pytestmark = pytest.mark.gpu

CQ_ERR_SCRATCH = 9


def _kv(seed, B, H, T, D=128):
    rng = np.random.default_rng(seed)
    k = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    v = np.cumsum(rng.standard_normal((B, H, T, D)) * 0.1, axis=2).astype(np.float16)
    return k, v


def _decode(cache, q, lens, T, max_T, noalloc):
    """One decode through the C ABI; returns (status, out)."""
    from chronoquant_mlx_amd import _lib
    L = _lib.load()
    B, nq, D = q.shape
    out = torch.full((B, nq, D), float("nan"), dtype=torch.float16, device=q.device)
    lens_ptr = None if lens is None else lens.data_ptr()
    sp = torch.cuda.current_stream().cuda_stream
    scale = D ** -0.5
    if noalloc:
        st = L.cq_decode_attn_noalloc(cache._descriptor(), q.data_ptr(), _lib.CQ_F16, nq, scale,
                                      lens_ptr, T, max_T, out.data_ptr(), _lib.CQ_F16, sp)
    else:
        H = cache._shape[1]
        need = L.cq_decode_workspace_size(B, H, nq, D, max_T)
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=q.device)
        st = L.cq_decode_attn(cache._descriptor(), q.data_ptr(), _lib.CQ_F16, nq, scale,
                              lens_ptr, T, max_T, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(),
                              ws.numel(), sp)
    torch.cuda.synchronize()
    return st, out


# (B, H, G, T, lens, strides): the c1 shape (32 splits of 512 tokens), then
# smaller inputs in the same scratch (fewer splits, a ragged batch on the
# balanced plan, the 16-head kernel at G = 8 and at strides that are not
# powers of two)
CASES = [
    (1, 8, 4, 16384, None, (32, 8)),
    (1, 8, 4, 3000, None, (32, 8)),
    (4, 8, 4, 2000, [2000, 1, 1057, 0], (32, 8)),
    (2, 2, 8, 700, None, (16, 4)),
    (2, 2, 4, 300, None, (5, 6)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_equals_workspace_entry(case):
    B, H, G, T, lens, (sk, sv) = CASES[case]
    k, v = _kv(100 + case, B, H, T)
    cache = build_gpu_cache(k, v, stride_k=sk, stride_v=sv)
    q = to_gpu(np.random.default_rng(200 + case).standard_normal((B, G * H, 128)))
    lt = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    st, ref = _decode(cache, q, lt, T, T, noalloc=False)
    assert st == 0
    for _ in range(2):  # the scratch keeps the last call's contents; counters return to 0
        st, got = _decode(cache, q, lt, T, T, noalloc=True)
        assert st == 0
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"case {case}"


def test_noalloc_two_calls_second_smaller():
    # two calls in a row on one scratch, the second with a smaller input
    outs = []
    for T in (16384, 1500):
        k, v = _kv(T, 1, 8, T)
        cache = build_gpu_cache(k, v, stride_k=32, stride_v=8)
        q = to_gpu(np.random.default_rng(T).standard_normal((1, 32, 128)))
        st, got = _decode(cache, q, None, T, T, noalloc=True)
        assert st == 0
        st, ref = _decode(cache, q, None, T, T, noalloc=False)
        assert st == 0
        outs.append((got, ref))
    for got, ref in outs:
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_rejects_shapes_beyond_the_scratch():
    # 64 ragged sequences bounded at 16384 tokens need 64 x 32 partial slots
    # x 32 heads x 520 bytes > 32 MiB: refused before any launch, output
    # untouched
    from chronoquant_mlx_amd import ChronoQuantCache, _lib
    B, H, T = 64, 8, 16384
    assert _lib.load().cq_decode_workspace_size(B, H, 32, 128, T) > (32 << 20)
    cache = ChronoQuantCache(stride_k=32, stride_v=8, capacity=T)
    x = torch.zeros(B, H, 1, 128, dtype=torch.float16, device="cuda")
    cache.update_and_fetch(x, x)
    q = torch.zeros(B, 32, 128, dtype=torch.float16, device="cuda")
    lens = torch.ones(B, dtype=torch.int32, device="cuda")
    st, out = _decode(cache, q, lens, 0, T, noalloc=True)
    assert st == CQ_ERR_SCRATCH, st
    assert torch.isnan(out.float()).all()
    assert "scratch" in _lib.status_string(st)


def test_noalloc_in_graph_replays():
    # captured once (after an eager call), replayed three times with eager
    # work of the library between the replays; every replay equals the eager
    # result
    from chronoquant_mlx_amd import _lib
    L = _lib.load()
    B, H, G, T = 2, 8, 4, 5000
    k, v = _kv(7, B, H, T)
    cache = build_gpu_cache(k, v, stride_k=64, stride_v=32, bits_v=3, dz_v=0.05)
    q = to_gpu(np.random.default_rng(8).standard_normal((B, G * H, 128)))
    st, ref = _decode(cache, q, None, T, T, noalloc=False)
    assert st == 0
    out = torch.empty_like(ref)
    desc = cache._descriptor()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        st = L.cq_decode_attn_noalloc(desc, q.data_ptr(), _lib.CQ_F16, G * H, 128 ** -0.5, None,
                                      T, T, out.data_ptr(), _lib.CQ_F16, side.cuda_stream)
        assert st == 0
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        st = L.cq_decode_attn_noalloc(desc, q.data_ptr(), _lib.CQ_F16, G * H, 128 ** -0.5, None,
                                      T, T, out.data_ptr(), _lib.CQ_F16, side.cuda_stream)
        assert st == 0
    other_k, other_v = _kv(9, 1, 8, 2500)
    other = build_gpu_cache(other_k, other_v, stride_k=32, stride_v=8)
    oq = to_gpu(np.random.default_rng(10).standard_normal((1, 32, 128)))
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        st, _ = _decode(other, oq, None, 2500, 2500, noalloc=True)  # eager work between
        assert st == 0
