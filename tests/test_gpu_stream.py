"""configs[3] at its workload: a ragged batch of 32 sequences (lengths drawn
uniform in [1024, 32768]), each step appending one token per sequence at its
own device-side position and then decoding one query per sequence over the
per-sequence lengths, the whole loop replayed as one HIP graph (the loop
bench.py times).

Reference: the per-token append of ChronoQuantCache (cache.py:87-129 via
update_and_fetch, :198-215) followed by the fused decode (attention.py:45-59);
each sequence b must behave exactly like an independent B=1 reference cache
of length T_b.  Checked per step against the oracle's restatement of the
reconstruct fallback (attention.py:61-74) and of the fused-kernel semantics
(kernels.py:79-228), and at the end bit for bit against the oracle's cache
state, for the shortest, the longest and two random sequences.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cqtest import ATOL, assert_close, assert_tight

pytestmark = pytest.mark.gpu


def _fallback_prefix(q_b, rk, rv, T, scale):
    """Reference fallback for one query per head over the first T tokens of
    the (prefix-closed) reconstruction rk, rv [H, T_final, D]."""
    return O.sdpa_fallback(q_b[:, None], np.ascontiguousarray(rk[:, :T]),
                           np.ascontiguousarray(rv[:, :T]), scale)[:, 0]


def test_c3_streaming_graph():
    from chronoquant_mlx_amd import ChronoQuantCache, _lib, synth
    cfg = synth.CONFIGS["c3"]
    B, H, D, nq = cfg.B, cfg.n_kv_heads, cfg.head_dim, cfg.n_q_heads
    steps = 256  # the loop bench.py times: 256 steps (every sequence crosses I-frames)
    lens = cfg.lengths()
    t_max = int(lens.max())
    cap = t_max + steps
    dev = torch.device("cuda")
    print(f"c3 stream: B={B} lens {lens.min()}..{t_max} steps={steps}", flush=True)

    import dataclasses
    kt, vt = synth.make_kv_device(dataclasses.replace(cfg, T=cap), cap, B, dev)
    # Initial fill: sequence b's first lens[b] tokens are its stream; the
    # rows past them (which the steps overwrite) hold other values, so an
    # append that wrote nothing could not pass.
    t_idx = torch.arange(cap, device=dev)[None, None, :, None]
    past = t_idx >= torch.as_tensor(lens, device=dev)[:, None, None, None]
    cache = ChronoQuantCache(stride_k=cfg.stride_k, stride_v=cfg.stride_v,
                             delta_bits_k=cfg.delta_bits_k, delta_bits_v=cfg.delta_bits_v,
                             dead_zone_k=cfg.dead_zone_k, dead_zone_v=cfg.dead_zone_v,
                             capacity=cap)
    cache.update_and_fetch(torch.where(past, -kt, kt), torch.where(past, -vt, vt))
    del past
    # step s appends token lens[b] + s of sequence b's own stream
    bi = torch.arange(B, device=dev)
    li = torch.as_tensor(lens, device=dev)
    k_steps = torch.stack([kt[bi, :, li + s] for s in range(steps)]).contiguous()  # [S, B, H, D]
    v_steps = torch.stack([vt[bi, :, li + s] for s in range(steps)]).contiguous()
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    q_steps = torch.randn(steps, B, nq, D, generator=g, device=dev).half()
    out_steps = torch.empty(steps, B, nq, D, dtype=torch.float16, device=dev)

    L = _lib.load()
    desc = cache._descriptor()
    off0 = torch.as_tensor(lens, dtype=torch.int32, device=dev)
    off, off1 = off0.clone(), off0 + 1
    need = L.cq_decode_workspace_size(B, H, nq, D, cap)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    strides = (ctypes.c_int64 * 3)(H * D, D, D)
    scale = D ** -0.5

    def step(s):
        sp = torch.cuda.current_stream().cuda_stream
        st = L.cq_append(desc, k_steps[s].data_ptr(), strides, v_steps[s].data_ptr(), strides,
                         _lib.CQ_F16, 1, off.data_ptr(), 0, sp)
        assert st == 0, _lib.status_string(st)
        st = L.cq_decode_attn(desc, q_steps[s].data_ptr(), _lib.CQ_F16, nq, scale, off1.data_ptr(),
                              0, cap, out_steps[s].data_ptr(), _lib.CQ_F16, ws.data_ptr(), need, sp)
        assert st == 0, _lib.status_string(st)
        off.add_(1)
        off1.add_(1)

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s in range(steps):
            step(s)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(off, off0 + steps)
    print("c3 stream: graph replayed", flush=True)

    rng = np.random.default_rng(3)
    order = np.argsort(lens)
    pick = [int(order[0]), int(order[-1])]
    pick += [int(b) for b in rng.choice([b for b in range(B) if b not in pick], 2, replace=False)]
    out = out_steps.float().cpu().numpy()
    q_np = q_steps.cpu().numpy()
    st = cache.state
    worst = 0.0
    for b in pick:
        n = int(lens[b]) + steps
        k_b = torch.cat([kt[b, :, :lens[b]], k_steps[:, b].transpose(0, 1)], dim=1).cpu().numpy()
        v_b = torch.cat([vt[b, :, :lens[b]], v_steps[:, b].transpose(0, 1)], dim=1).cpu().numpy()
        ck = O.OracleComponent(H, D, cfg.stride_k, cfg.delta_bits_k, cfg.dead_zone_k, capacity=n)
        cv = O.OracleComponent(H, D, cfg.stride_v, cfg.delta_bits_v, cfg.dead_zone_v, capacity=n)
        ck.append(k_b)
        cv.append(v_b)
        # final state of sequence b, bit for bit (the active prefix of length n)
        for i, comp in ((0, ck), (1, cv)):
            kf, pk, sc = comp.active()
            g_kf = st[i][b][:, :kf.shape[1]].cpu().numpy()
            g_pk = st[2 + 2 * i][b][:, :pk.shape[1]].cpu().numpy()
            g_sc = st[3 + 2 * i][b][:, :sc.shape[1]].cpu().numpy()
            assert np.array_equal(g_kf.view(np.uint16), kf.view(np.uint16)), f"b={b} keyframes[{i}]"
            assert np.array_equal(g_pk, pk), f"b={b} packed[{i}]"
            assert np.array_equal(g_sc.view(np.uint16), sc.view(np.uint16)), f"b={b} scales[{i}]"
        rk, rv = ck.reconstruct(), cv.reconstruct()
        # every 16th step (and the first and last) against the oracle
        for s in sorted(set(range(0, steps, 16)) | {1, steps - 1}):
            T = int(lens[b]) + s + 1
            ref = _fallback_prefix(q_np[s, b], rk, rv, T, scale)
            e, _ = assert_close(out[s, b], ref, what=f"b={b} step={s} T={T}")
            worst = max(worst, e)
            assert_tight(out[s, b], O.sdpa_fused(q_np[s, b], ck, cv, scale, T=T),
                         what=f"b={b} step={s} T={T}")
    # the bar also holds as a plain max-abs (outputs reach [2, 4), where one
    # fp16 ulp is 1.95e-3)
    assert worst <= ATOL, worst
    print(f"c3 stream: sequences {pick} bit-exact, worst max-abs {worst:.2e}", flush=True)
