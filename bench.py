"""Benchmark of the ChronoQuant decode hot path on one MI355X.

A step is one fused dequant-SDPA decode of one attention layer (one query
token per sequence over the compressed cache) at the workload BASELINE.json's
metric is quoted on: configs[1], GQA 32q/8kv, head_dim 128, 16K context,
B=1, strides 32/8, INT4 K and V residuals.

* The cache is built once by the append kernel from the seeded AR(1)
  generator, then cloned into enough replicas (>= 8, and >= 4.5 x the 256 MB
  Infinity Cache) that the steps, which cycle the replicas, read their bytes
  from HBM.
* The K timed steps are captured once in a HIP graph and replayed, so the
  GPU runs them back to back; HIP events on the launch stream bracket the
  timed replay (after W warmup steps).
* value = algorithmic bytes per step (the reference's nbytes of the cache +
  Q + O) / time per step, in GB/s; roofline.frac = value / 8 TB/s.
* The uncompressed fp16 flash decode over the same K/V (cq_fp16_decode_attn)
  is timed the same way; cpu_baseline times the CPU oracle's restatement of
  the reference's decode (reconstruct K/V + fallback SDPA) on host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
# Timed steps cycle through at least this many times MALL_BYTES of distinct
# caches, and through at least 8 replicas.  Decode times fall 6-10 % when the
# cycle spans only 2-2.3 x the Infinity Cache (part of each step's bytes are
# still held there) and reach their plateau from about 4 x on.
REPLICA_SPAN = 4.5


def replica_count(nbytes, floor=8):
    """Replicas of an nbytes cache (or K/V pair) the timed steps cycle."""
    return max(floor, int(np.ceil(REPLICA_SPAN * MALL_BYTES / nbytes)))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_cache(cfg, dev):
    import torch

    from chronoquant_mlx_amd import ChronoQuantCache, synth
    k, v = synth.make_kv(cfg)
    cache = ChronoQuantCache(stride_k=cfg.stride_k, stride_v=cfg.stride_v,
                             delta_bits_k=cfg.delta_bits_k, delta_bits_v=cfg.delta_bits_v,
                             dead_zone_k=cfg.dead_zone_k, dead_zone_v=cfg.dead_zone_v,
                             capacity=cfg.T)
    kt = torch.from_numpy(k).to(dev)
    vt = torch.from_numpy(v).to(dev)
    cache.update_and_fetch(kt, vt)
    torch.cuda.synchronize()
    return cache, k, v, kt, vt


def build_cache_device(cfg, dev, capacity=None, dense=False):
    """Cache filled from the on-GPU generator (workloads too large for the
    host generator); same AR(1) statistics, different random streams.
    dense: 2- and 3-bit residual rows stored at their width (dense_residuals)."""
    import torch

    from chronoquant_mlx_amd import ChronoQuantCache, synth
    kt, vt = synth.make_kv_device(cfg, cfg.T, cfg.B, dev)
    cache = ChronoQuantCache(stride_k=cfg.stride_k, stride_v=cfg.stride_v,
                             delta_bits_k=cfg.delta_bits_k, delta_bits_v=cfg.delta_bits_v,
                             dead_zone_k=cfg.dead_zone_k, dead_zone_v=cfg.dead_zone_v,
                             capacity=capacity or cfg.T, dense_residuals=dense)
    cache.update_and_fetch(kt, vt)
    torch.cuda.synchronize()
    return cache, kt, vt


def clone_cache(cache):
    import copy
    c = copy.copy(cache)
    c._kf = {x: cache._kf[x].clone() for x in ("k", "v")}
    c._pk = {x: cache._pk[x].clone() for x in ("k", "v")}
    c._sc = {x: cache._sc[x].clone() for x in ("k", "v")}
    return c


def whole_cycles(steps, n):
    """Launches timed for `steps` requested over n replicas: whole cycles of
    the replicas (at least one), so that every replica counted in the
    distinct bytes is read the same number of times."""
    return max(1, -(-steps // n)) * n


# launches the last time_graph / time_eager call timed (whole replica cycles)
LAST_LAUNCHES = {"n": 0}


def time_graph(launch_fns, steps, warmup, stream):
    """Capture whole cycles of launch_fns (at least `steps` launches) in a
    graph; replay once for warmup, then time one replay with events on
    `stream`.  Returns ms per launch over the launches captured."""
    import torch
    n = len(launch_fns)
    launches = whole_cycles(steps, n)
    # warm up on the capture stream: the library sizes that stream's split
    # workspace outside capture
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            launch_fns[i % n]()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(launches):
            launch_fns[i % n]()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        g.replay()
        e1.record(stream)
    e1.synchronize()
    LAST_LAUNCHES["n"] = launches
    return e0.elapsed_time(e1) / launches  # ms per launch


def time_eager(launch_fns, steps, warmup, stream):
    """Launch whole cycles of launch_fns (at least `steps` launches) without a
    graph, bracketed by events on `stream` (for profilers that count per
    dispatch).  Returns ms per launch."""
    import torch
    n = len(launch_fns)
    launches = whole_cycles(steps, n)
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            launch_fns[i % n]()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(launches):
            launch_fns[i % n]()
        e1.record(stream)
    e1.synchronize()
    LAST_LAUNCHES["n"] = launches
    return e0.elapsed_time(e1) / launches


def cycle_record(algo_bytes, replicas):
    """What the timed launches read: the replicas' distinct bytes and their
    ratio to the 256 MB Infinity Cache, and the launches timed."""
    distinct = int(algo_bytes) * int(replicas)
    return {"replicas": int(replicas), "launches_timed": LAST_LAUNCHES["n"],
            "distinct_bytes_cycled": distinct,
            "distinct_bytes_over_infinity_cache": round(distinct / MALL_BYTES, 2)}


def copy_calibration(dev, nbytes=256 << 20, reps=4):
    """Plain device copies of known size: the reference reading of the
    FETCH_SIZE / WRITE_SIZE counters (each copy reads and writes nbytes)."""
    import torch
    src = torch.empty(nbytes // 2, dtype=torch.float16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy calibration: {reps} copies of {nbytes} bytes")


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_g4_c1_traffic.txt")


def kernel_source_hash():
    import hashlib
    h = hashlib.sha256()
    for f in ("cq_decode_g4.hip", "cq_mfma_common.h", "cq_decode_common.h", "cq_plan.h",
              "cq_device.h"):
        with open(os.path.join(ROOT, "chronoquant_mlx_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


PREFILL_COUNTERS_FILE = os.path.join(ROOT, "profiles", "prefill_c4_chunk_counters.txt")


def prefill_source_hash():
    import hashlib
    h = hashlib.sha256()
    for f in ("cq_prefill.hip", "cq_decode_common.h", "cq_plan.h", "cq_device.h"):
        with open(os.path.join(ROOT, "chronoquant_mlx_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_prefill_mfma_busy():
    """MFMA busy fraction of the prefill kernel (SQ_VALU_MFMA_BUSY_CYCLES per
    SIMD over the dispatch's cycles) from the committed rocprofv3 --pmc
    summary, if it was measured on the current kernel source."""
    try:
        with open(PREFILL_COUNTERS_FILE) as fh:
            kv = dict(line.split("=", 1) for line in fh.read().splitlines() if "=" in line
                      and not line.startswith((" ", "#", "rocprofv3")))
    except OSError:
        return None
    kv = {a.strip(): b.strip() for a, b in kv.items()}
    if kv.get("kernel_source_sha256_16") != prefill_source_hash():
        return None
    return float(kv["mfma_busy_frac"])


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if it
    was measured on the current kernel source and this workload."""
    try:
        with open(TRAFFIC_FILE) as fh:
            kv = dict(line.split("=", 1) for line in fh.read().splitlines() if "=" in line
                      and not line.startswith((" ", "#", "rocprofv3")))
    except OSError:
        return None
    kv = {a.strip(): b.strip() for a, b in kv.items()}
    if kv.get("kernel_source_sha256_16") != kernel_source_hash() or kv.get("workload") != workload:
        return None
    return int(kv["traffic_bytes_per_launch"])


def time_torch_sdpa(cfg, kvs, q, scale, stream, steps, warmup, timer, check_against=None):
    """torch.nn.functional.scaled_dot_product_attention as an independent fp16
    decode over the same uncompressed K/V replicas, on each backend that runs
    this shape without the math fallback (flash, memory-efficient) and in
    two layouts: GQA decode as G query rows per kv head (q [B, H, G, D]
    against k, v [B, H, T, D], no mask: K/V read once) and torch's own
    enable_gqa (q [B, nq, 1, D]).  Returns every timing and the fastest."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    B, nq, D = q.shape
    H = cfg.n_kv_heads
    layouts = {"gqa_rows": (q.reshape(B, H, nq // H, D), {}),
               "enable_gqa": (q.reshape(B, nq, 1, D), {"enable_gqa": True})}
    runs, best = [], None
    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        for lname, (qq, kw) in layouts.items():
            rec = {"backend": backend.name, "layout": lname}
            try:
                with sdpa_kernel([backend]):
                    o = F.scaled_dot_product_attention(qq, kvs[0][0], kvs[0][1], scale=scale, **kw)
                torch.cuda.synchronize()
            except RuntimeError as e:
                rec["error"] = str(e).splitlines()[0][:160]
                runs.append(rec)
                continue

            def mk(kk, vv, backend=backend, qq=qq, kw=kw):
                def f():
                    with sdpa_kernel([backend]):
                        F.scaled_dot_product_attention(qq, kk, vv, scale=scale, **kw)
                return f

            ms = timer([mk(a, b) for a, b in kvs], steps, warmup, stream)
            rec["us_per_layer"] = round(ms * 1e3, 3)
            if check_against is not None:
                rec["max_abs_diff_vs_cq_fp16_decode"] = float(
                    (o.reshape(B, nq, D).float() - check_against.float()).abs().max())
            runs.append(rec)
            if best is None or rec["us_per_layer"] < best["us_per_layer"]:
                best = rec
    return {"us_per_layer": None if best is None else best["us_per_layer"],
            "fastest": best, "runs": runs}


def time_decode_config(name, dev, stream, steps, warmup, timer, device_gen, dense=False):
    """Fused decode of one configuration (full context, every sequence at T):
    us/layer and algorithmic GB/s over cycled cache replicas.  dense: the
    cache's 2- and 3-bit residual rows at their width (algorithmic bytes are
    then that cache's nbytes + Q + O)."""
    import torch

    from chronoquant_mlx_amd import _lib, synth
    cfg = synth.CONFIGS[name]
    if device_gen:
        cache, kt, vt = build_cache_device(cfg, dev, dense=dense)
    else:
        assert not dense
        cache, _, _, kt, vt = build_cache(cfg, dev)
    del kt, vt
    q = torch.randn(cfg.B, cfg.n_q_heads, cfg.head_dim, device=dev).half()
    scale = cfg.head_dim ** -0.5
    algo = synth.algorithmic_decode_bytes(cfg)
    if dense:
        algo = cache.nbytes + 2 * q.numel() * 2
    reps = replica_count(cache.nbytes)
    caches = [cache] + [clone_cache(cache) for _ in range(reps - 1)]
    out = torch.empty(cfg.B, cfg.n_q_heads, cfg.head_dim, dtype=torch.float16, device=dev)
    L = _lib.load()
    ws = caches[0]._decode_workspace(cfg.n_q_heads)
    descs = [c._descriptor() for c in caches]

    def mk(desc):
        def f():
            st = L.cq_decode_attn(desc, q.data_ptr(), _lib.CQ_F16, cfg.n_q_heads, scale, None,
                                  cfg.T, cfg.T, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(),
                                  ws.numel(), torch.cuda.current_stream().cuda_stream)
            assert st == 0, _lib.status_string(st)
        return f

    ms = timer([mk(d) for d in descs], steps, warmup, stream)
    gbs = algo / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms * 1e3:.2f} us/layer, {gbs:.0f} GB/s")
    res = {"workload": f"B={cfg.B} GQA {cfg.n_q_heads}q/{cfg.n_kv_heads}kv T={cfg.T} strides "
                       f"{cfg.stride_k}/{cfg.stride_v} bits {cfg.delta_bits_k}/{cfg.delta_bits_v} "
                       f"dz {cfg.dead_zone_k}/{cfg.dead_zone_v}",
           "us_per_layer": round(ms * 1e3, 3), "GBps": round(gbs, 1),
           "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": algo,
           **cycle_record(algo, reps),
           "data": "on-GPU AR(1) generator" if device_gen else "seeded AR(1)"}
    if dense:
        res["workload"] += "; dense 3-bit V rows (48 B) in HBM"
    del caches, cache
    torch.cuda.empty_cache()
    return res


def time_streaming(name, dev, stream, n_steps=256):
    """a ragged batch, each step appends one token per sequence
    (I-frame every stride, else quantise + pack against the anchor) and runs
    the fused decode over the per-sequence lengths; the n_steps steps are one
    HIP graph, timed once after an untimed replay.  Each step does this for
    every one of a few identical layer caches in turn (as a model's layers
    would), so that a decode reads its cache from HBM; figures are per layer
    step."""
    import torch

    from chronoquant_mlx_amd import _lib, synth
    cfg = synth.CONFIGS[name]
    B, H, D, nq = cfg.B, cfg.n_kv_heads, cfg.head_dim, cfg.n_q_heads
    lens = cfg.lengths()
    t_max = int(lens.max())
    cap = t_max + n_steps
    import dataclasses
    gcfg = dataclasses.replace(cfg, T=cap)
    cache, kt, vt = build_cache_device(gcfg, dev, capacity=cap)
    # every sequence holds t_max tokens; sequence b continues at lens[b]
    algo = int(np.mean([synth.algorithmic_decode_bytes(cfg, lens + s + 1) for s in range(n_steps)]))
    n_layers = replica_count(algo, floor=1)  # by the bytes a decode reads
    caches = [cache] + [clone_cache(cache) for _ in range(n_layers - 1)]
    descs = [c._descriptor() for c in caches]
    L = _lib.load()
    off0 = torch.tensor(lens, dtype=torch.int32, device=dev)
    off = off0.clone()
    off1 = off0 + 1
    q = torch.randn(B, nq, D, device=dev).half()
    out = torch.empty(B, nq, D, dtype=torch.float16, device=dev)
    need = L.cq_decode_workspace_size(B, H, nq, D, cap)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    ks = (ctypes.c_int64 * 3)(*kt.stride()[:3])
    vs = (ctypes.c_int64 * 3)(*vt.stride()[:3])
    scale = D ** -0.5

    def step(s):
        sp = torch.cuda.current_stream().cuda_stream
        kn, vn = kt[:, :, t_max + s - n_steps], vt[:, :, t_max + s - n_steps]
        for desc in descs:
            st = L.cq_append(desc, kn.data_ptr(), ks, vn.data_ptr(), vs, _lib.CQ_F16, 1,
                             off.data_ptr(), 0, sp)
            assert st == 0, _lib.status_string(st)
            st = L.cq_decode_attn(desc, q.data_ptr(), _lib.CQ_F16, nq, scale, off1.data_ptr(), 0,
                                  cap, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(), need, sp)
            assert st == 0, _lib.status_string(st)
        off.add_(1)
        off1.add_(1)

    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for s in range(n_steps):
            step(s)
    def reset():
        off.copy_(off0)
        off1.copy_(off0 + 1)
        torch.cuda.synchronize()
    reset()
    g.replay()
    reset()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        g.replay()
        e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / (n_steps * n_layers)
    gbs = algo / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms * 1e3:.2f} us/step (append + decode), {gbs:.0f} GB/s")
    res = {"workload": f"B={B} ragged T_b~U[{cfg.ragged_min},{cfg.T}] GQA {nq}q/{H}kv strides "
                       f"{cfg.stride_k}/{cfg.stride_v}; {n_steps} steps of append(1 token/seq) + "
                       f"fused decode on each of {n_layers} layer caches, one HIP graph",
           "us_per_step": round(ms * 1e3, 3), "GBps": round(gbs, 1),
           "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": algo,
           "layers": n_layers, "data": "on-GPU AR(1) generator"}
    del g, cache, caches, kt, vt
    torch.cuda.empty_cache()
    return res


def time_prefill(dev, stream, steps, T=8192, L=512):
    """Chunked-prefill attention (cq_prefill_attn) on configs[4]'s shape: the
    last L-token chunk of a T-token prompt, GQA 32q/8kv, Full-Throttle V3
    codec; against the reconstruct fallback (cq_reconstruct + dense torch
    attention) on the same call."""
    import dataclasses

    import torch

    from chronoquant_mlx_amd import attention as A
    from chronoquant_mlx_amd import synth
    from chronoquant_mlx_amd.kernels import chronoquant_prefill_kernel
    cfg = dataclasses.replace(synth.CONFIGS["ftv3_16k"], T=T)
    cache, kt, vt = build_cache_device(cfg, dev)
    del kt, vt
    nq, D, H = cfg.n_q_heads, cfg.head_dim, cfg.n_kv_heads
    q = torch.randn(1, nq, L, D, device=dev).half()
    scale = D ** -0.5
    # causal FLOPs: QK^T and PV, 2 flops per MAC, query i sees T - L + i + 1 keys
    keys = L * (T - L) + L * (L + 1) // 2
    flops = 4 * D * nq * keys
    ms = time_graph([lambda: chronoquant_prefill_kernel(q, cache, scale, causal=True)],
                    steps, 3, stream)
    A.PREFILL_KERNEL = False
    try:
        # eager: the fallback creates small host-side tensors (not capturable)
        ms_fb = time_eager([lambda: A.chronoquant_sdpa(q, None, None, cache, scale, mask="causal")],
                           max(5, steps // 10), 2, stream)
    finally:
        A.PREFILL_KERNEL = True
    tf = flops / (ms * 1e-3) / 1e12
    log(f"[bench] prefill T={T} L={L}: {ms * 1e3:.1f} us ({tf:.1f} TFLOP/s), "
        f"reconstruct fallback {ms_fb * 1e3:.1f} us")
    res = {"workload": f"B=1 GQA {nq}q/{H}kv D={D}: last {L}-token chunk of a {T}-token prompt, "
                       f"causal, strides {cfg.stride_k}/{cfg.stride_v} bits "
                       f"{cfg.delta_bits_k}/{cfg.delta_bits_v}",
           "us_per_call": round(ms * 1e3, 2), "TFLOPs": round(tf, 2),
           "frac_of_fp16_mfma_peak": round(tf / 2500.0, 4), "flops_per_call": flops,
           "reconstruct_fallback_us": round(ms_fb * 1e3, 2),
           "speedup_vs_fallback": round(ms_fb / ms, 2),
           # from profiles/prefill_c4_chunk_counters.txt (null when the kernel
           # source changed since it was measured)
           "mfma_busy_frac": measured_prefill_mfma_busy()}
    del cache
    torch.cuda.empty_cache()
    return res


def time_e2e(dev, prompt_len=8192, n_new=512, chunk=512):
    """random-init Qwen-style decoder (32 layers, hidden 4096, GQA
    32/8, SwiGLU 12288, RoPE 1e6, vocab 151936, bf16 N(0, 0.02)) with
    Full-Throttle V3 ChronoQuant caches in every layer via apply(): the
    prompt in chunk-token prefill chunks, then n_new greedy tokens (decode
    steps captured as one HIP graph, positions on the device)."""
    import torch

    from chronoquant_mlx_amd import create_full_throttle_caches, patch
    from chronoquant_mlx_amd.models.qwen import ModelArgs, generate, random_model
    args = ModelArgs()
    model = random_model(args, device=dev, seed=0)
    n_params = sum(p.numel() for p in model.parameters())
    patch.apply()
    try:
        prompt = torch.randint(0, args.vocab_size, (1, prompt_len),
                               generator=torch.Generator().manual_seed(0)).to(dev)
        # warm-up on a short prompt (kernel loading, library handles, workspaces)
        generate(model, create_full_throttle_caches(model), prompt[:, :chunk], 4, chunk)
        caches = create_full_throttle_caches(model)
        toks, t_pre, t_dec = generate(model, caches, prompt, n_new, chunk)
    finally:
        patch.revert()
    total_tokens = prompt_len + n_new - 1
    kv = sum(c.nbytes for c in caches)
    fp16_kv = 2 * args.num_hidden_layers * args.num_key_value_heads * args.head_dim * 2
    res = {"workload": f"Qwen-style decoder {args.num_hidden_layers} layers hidden "
                       f"{args.hidden_size} GQA {args.num_attention_heads}/{args.num_key_value_heads} "
                       f"SwiGLU {args.intermediate_size} vocab {args.vocab_size}, bf16 random "
                       f"N(0,0.02) ({n_params / 1e9:.2f}B params); {prompt_len}-token prompt in "
                       f"{chunk}-token chunks + {n_new} greedy tokens; Full-Throttle V3 caches",
           "prefill_tokens_per_s": round(prompt_len / t_pre, 1),
           "decode_tokens_per_s": round((n_new - 1) / t_dec, 2),
           "decode_ms_per_token": round(t_dec / (n_new - 1) * 1e3, 3),
           "end_to_end_tokens_per_s": round((prompt_len + n_new - 1) / (t_pre + t_dec), 1),
           "kv_bytes_per_token": round(kv / total_tokens, 1),
           "fp16_kv_bytes_per_token": fp16_kv,
           "weight_bytes": int(sum(p.numel() * p.element_size() for p in model.parameters())),
           "data": "uniform random token ids, seed 0"}
    log(f"[bench] c4: prefill {res['prefill_tokens_per_s']} tok/s, decode "
        f"{res['decode_tokens_per_s']} tok/s ({res['decode_ms_per_token']} ms/token), "
        f"KV {res['kv_bytes_per_token']} B/token (fp16 {fp16_kv})")
    del model, caches
    torch.cuda.empty_cache()
    return res


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> tuple[int, str]:
    """Threads for the CPU baseline: the process's CPU affinity, capped by
    OMP_NUM_THREADS when that is set (the GPU box sets it to its CPU share
    per GPU, 16)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < aff:
        return int(omp), f"OMP_NUM_THREADS={omp} (the host's CPU share for this GPU) of {aff} in affinity"
    return aff, f"all {aff} CPUs in the process affinity"


def cpu_baseline_config(cfg, k, v, q, threads, runs=50, warmup=3, max_s=10.0, fallback_runs=3):
    """The reference's per-layer decode work on the host CPU (oracle/): one
    token's append (codec + INT4 pack + I-frame, cache.py:87-129 with
    codec.py:23-65 and kernels.py:34-54) and the fused compressed-cache
    attention of kernels.py:79-228 in fp32 (oracle/cq_cpu_baseline.c:
    OpenMP over kv-head x key-chunk tasks, AVX2), over the same T tokens the
    GPU decodes; medians of `runs` after `warmup` (fewer if max_s runs
    out).  Also times, `fallback_runs` times, the reference's other decode
    route: reconstruct K/V (cache.py:131-160) and the fallback SDPA
    (attention.py:61-74), the oracle's binary64-accumulating restatement."""
    from oracle import oracle as O
    O.set_threads(threads)
    H, D, T = cfg.n_kv_heads, cfg.head_dim, cfg.T
    n_app = 23
    ck = O.OracleComponent(H, D, cfg.stride_k, cfg.delta_bits_k, cfg.dead_zone_k,
                           capacity=T + n_app)
    cv = O.OracleComponent(H, D, cfg.stride_v, cfg.delta_bits_v, cfg.dead_zone_v,
                           capacity=T + n_app)
    ck.append(k[0])
    cv.append(v[0])
    # append: the next tokens of the stream (AR(1) continuation = the last
    # token, so residuals stay of the stream's size), one at a time
    tok = np.ascontiguousarray(k[0][:, -1:])
    vtok = np.ascontiguousarray(v[0][:, -1:])
    t_app = []
    for i in range(n_app):
        t0 = time.perf_counter()
        ck.append(tok)
        cv.append(vtok)
        t_app.append(time.perf_counter() - t0)
    t_app = t_app[3:]
    t_att = []
    out = None
    t_start = time.perf_counter()
    for i in range(runs + warmup):
        t0 = time.perf_counter()
        out = O.fused_decode_f32(q[0], ck, cv, D ** -0.5, T=T)
        if i >= warmup:
            t_att.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > max_s and len(t_att) >= 5:
            break
    t_fb = []
    if fallback_runs:
        Tn = ck.offset
        scratch = (np.empty((H, Tn, D), np.uint16), np.empty((H, Tn, D), np.uint16))
        O.decode_step(q[0], ck, cv, D ** -0.5, scratch)
        for i in range(fallback_runs):
            t0 = time.perf_counter()
            O.decode_step(q[0], ck, cv, D ** -0.5, scratch)
            t_fb.append(time.perf_counter() - t0)
    return (float(np.median(t_app)), float(np.median(t_att)), len(t_att), out,
            float(np.median(t_fb)) if t_fb else None)


def cpu_baseline(q_np_c1, ref_c1, algo_c1):
    """cpu_baseline for the JSON line: c1 (the metric's workload) and c0.
    ref_c1: the GPU's c1 output (fp32 [nq, D]) to compare with, or None."""
    from chronoquant_mlx_amd import synth
    threads, why = cpu_threads()
    res = {}
    for name in ("c1", "c0"):
        cfg = synth.CONFIGS[name]
        k, v = synth.make_kv(cfg)
        q = q_np_c1 if name == "c1" else synth.make_q(cfg)
        t_app, t_att, n, out, t_fb = cpu_baseline_config(cfg, k, v, q, threads)
        algo = synth.algorithmic_decode_bytes(cfg)
        res[name] = {"append_us": round(t_app * 1e6, 2), "attention_us": round(t_att * 1e6, 1),
                     "step_us": round((t_app + t_att) * 1e6, 1),
                     "GBps": round(algo / (t_app + t_att) / 1e9, 3), "runs": n,
                     "context": cfg.T,
                     "fallback_attention_us": None if t_fb is None else round(t_fb * 1e6, 1)}
        log(f"[bench] CPU {name}: append {t_app * 1e6:.1f} us + fused attention "
            f"{t_att * 1e6:.0f} us on {threads} threads (reconstruct + fallback SDPA "
            f"{(t_fb or 0) * 1e6:.0f} us)")
        if name == "c1" and ref_c1 is not None:
            res[name]["gpu_vs_cpu_max_abs_diff"] = float(
                np.abs(ref_c1.astype(np.float32) - out.astype(np.float32)).max())
    c1 = res["c1"]
    return {"value": c1["GBps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "threads_rule": why,
            "sample": "the reference's per-layer decode step on the host CPU (oracle/): append of "
                      "one token (codec + pack, oracle/cq_oracle.c) and the fused compressed-cache "
                      "attention of kernels.py:79-228 in fp32 (oracle/cq_cpu_baseline.c: OpenMP "
                      "kv-head x key-chunk tasks, AVX2/F16C) over the full c1 / c0 cache, medians "
                      f"of up to 50 runs after 3 warm-ups; value = c1 algorithmic bytes ({algo_c1}) "
                      "/ (append + attention).  fallback_attention_us: reconstruct K/V + fallback "
                      "SDPA (binary64 sums), the reference's unfused route, 3 runs",
            "configs": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--replicas", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fp16-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="launch without a HIP graph (for rocprofv3 --pmc passes)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run plain 256 MiB copies (counter scale reference)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the supplementary ftv3_16k / c2 / c3 / prefill / c4 measurements")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end configs[4] model run")
    ap.add_argument("--e2e-only", action="store_true",
                    help="run only the configs[4] model and print its figures (for profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the chunked-prefill measurement and print its figures "
                         "(for profiling)")
    ap.add_argument("--split-tokens", type=int, default=0,
                    help="force the decode's split length (tokens, a multiple of 64) through "
                         "CQ_DECODE_SPLIT_TOKENS, for split-count sweeps")
    args = ap.parse_args()
    if args.split_tokens:
        # read by libchronoquant.so at its first decode plan
        os.environ["CQ_DECODE_SPLIT_TOKENS"] = str(args.split_tokens)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                                   "(the path shards by sequence / kv head with no exchange, "
                                   "but no multi-GPU figure is produced)"}))
        sys.exit(2)

    import torch

    from chronoquant_mlx_amd import _lib, synth
    from chronoquant_mlx_amd.kernels import chronoquant_sdpa_cache_kernel

    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    if args.e2e_only:
        print(json.dumps({"c4": time_e2e(dev)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": time_prefill(dev, torch.cuda.Stream(dev), args.steps)}),
              flush=True)
        return
    stream = torch.cuda.Stream(dev)
    log(f"[bench] building {cfg.name} cache (T={cfg.T}, B={cfg.B})")
    cache, k, v, kt, vt = build_cache(cfg, dev)
    q_np = synth.make_q(cfg)
    q = torch.from_numpy(q_np).to(dev)
    scale = cfg.head_dim ** -0.5
    algo_bytes = synth.algorithmic_decode_bytes(cfg)
    assert cache.nbytes + 2 * q.numel() * 2 == algo_bytes, (cache.nbytes, algo_bytes)

    reps = args.replicas or replica_count(cache.nbytes)
    caches = [cache] + [clone_cache(cache) for _ in range(reps - 1)]
    out = torch.empty(cfg.B, cfg.n_q_heads, cfg.head_dim, dtype=torch.float16, device=dev)
    L = _lib.load()
    ws = caches[0]._decode_workspace(cfg.n_q_heads)
    descs = [c._descriptor() for c in caches]

    def mk(desc):
        def f():
            st = L.cq_decode_attn(desc, q.data_ptr(), _lib.CQ_F16, cfg.n_q_heads, scale, None,
                                  cfg.T, cfg.T, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(),
                                  ws.numel(), torch.cuda.current_stream().cuda_stream)
            assert st == 0, _lib.status_string(st)
        return f

    log(f"[bench] {reps} replicas x {cache.nbytes / 1e6:.1f} MB; timing {args.steps} steps")
    timer = time_eager if args.eager else time_graph
    ms = timer([mk(d) for d in descs], args.steps, args.warmup, stream)
    gbs = algo_bytes / (ms * 1e-3) / 1e9
    # correctness of the timed kernel against the eager call
    ref = chronoquant_sdpa_cache_kernel(q, cache, scale)
    torch.cuda.synchronize()
    log(f"[bench] decode {ms * 1e3:.2f} us/layer, {gbs:.0f} GB/s")

    result = {
        "metric": "dequant-SDPA decode µs/layer + effective HBM GB/s (% peak), GQA 32/8 @16K",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "us_per_layer": round(ms * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name}: B={cfg.B} GQA {cfg.n_q_heads}q/{cfg.n_kv_heads}kv "
                               f"D={cfg.head_dim} T={cfg.T} strides {cfg.stride_k}/{cfg.stride_v} "
                               f"INT{cfg.delta_bits_k}/INT{cfg.delta_bits_v} (seeded AR(1) fp16 K/V)",
                   "algorithmic_bytes_per_step": algo_bytes,
                   **cycle_record(algo_bytes, reps)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(cfg.name)},
    }
    if args.eager:
        result["config"]["launch"] = "eager"
    if args.split_tokens:
        result["config"]["split_tokens"] = args.split_tokens
    if args.copy_calibration:
        copy_calibration(dev)

    if not args.no_fp16_baseline:
        H, D, T = cfg.n_kv_heads, cfg.head_dim, cfg.T
        fp16_bytes = 2 * cfg.B * H * T * D * 2 + 2 * q.numel() * 2
        reps16 = replica_count(fp16_bytes)
        kvs = [(kt, vt)] + [(kt.clone(), vt.clone()) for _ in range(reps16 - 1)]
        need = L.cq_decode_workspace_size(cfg.B, H, cfg.n_q_heads, D, T)
        ws16 = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)

        def mk16(kk, vv):
            def f():
                st = L.cq_fp16_decode_attn(kk.data_ptr(), vv.data_ptr(), T, cfg.B, H, D,
                                           q.data_ptr(), _lib.CQ_F16, cfg.n_q_heads, scale, None,
                                           T, T, out.data_ptr(), _lib.CQ_F16, ws16.data_ptr(),
                                           ws16.numel(), torch.cuda.current_stream().cuda_stream)
                assert st == 0, _lib.status_string(st)
            return f

        ms16 = timer([mk16(a, b) for a, b in kvs], args.steps, args.warmup, stream)
        log(f"[bench] fp16 flash decode {ms16 * 1e3:.2f} us/layer")
        mk16(*kvs[0])()  # cq_fp16_decode_attn's output on replica 0, for the cross-check
        torch.cuda.synchronize()
        out16 = out.clone()
        tsd = time_torch_sdpa(cfg, kvs, q, scale, stream, args.steps, args.warmup, timer,
                              check_against=out16)
        log(f"[bench] torch SDPA fp16 decode: {tsd}")
        cands = [ms16 * 1e3] + ([tsd["us_per_layer"]] if tsd.get("us_per_layer") else [])
        best = min(cands)
        result["fp16_baseline"] = {"us_per_layer": round(ms16 * 1e3, 3),
                                   "GBps": round(fp16_bytes / (ms16 * 1e-3) / 1e9, 1),
                                   "kernel": "cq_fp16_decode_attn (this library's fp16 split-K decode)",
                                   "torch_sdpa": tsd,
                                   "fastest_us_per_layer": round(best, 3),
                                   "speedup_of_compressed": round(best / (ms * 1e3), 3)}

    if not args.no_extra:
        extra = {}
        extra["ftv3_16k"] = time_decode_config("ftv3_16k", dev, stream, args.steps, args.warmup,
                                               timer, device_gen=False)
        if "fp16_baseline" in result:  # same K/V shape as the main workload
            extra["ftv3_16k"]["speedup_vs_fp16"] = round(
                result["fp16_baseline"]["fastest_us_per_layer"]
                / extra["ftv3_16k"]["us_per_layer"], 3)
        extra["c2"] = time_decode_config("c2", dev, stream, args.steps, args.warmup, timer,
                                         device_gen=True)
        extra["c2_dense"] = time_decode_config("c2", dev, stream, args.steps, args.warmup, timer,
                                               device_gen=True, dense=True)
        extra["c3"] = time_streaming("c3", dev, stream)
        extra["prefill"] = time_prefill(dev, stream, 50)
        if not args.no_e2e:
            extra["c4"] = time_e2e(dev)
        result["extra"] = extra

    if not args.no_cpu_baseline and cfg.name == "c1":
        log("[bench] CPU baseline (append + fused fp32 attention on the host CPU)")
        result["cpu_baseline"] = cpu_baseline(q_np, ref[0].float().cpu().numpy(), algo_bytes)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
