"""Where the time of one B=1 fused decode goes (diagnostic).

    python -m chronoquant_mlx_amd.build --phases
    python -m chronoquant_mlx_amd.phase_times [--config c1] [--launches 200] [--fp16]

Runs the decode of a benchmark configuration with libchronoquant_phases.so,
the library built with -DCQ_PHASE_TIMES: wave 0 of every workgroup of a
fold-record launch writes the device clock (s_memrealtime, 100 MHz, common
to all CUs) at six points into the launch's otherwise unused split-partial
area:

    0 workgroup started      1 first chunk's loads issued
    2 q table ready          3 wave 0's chunk computed (one-chunk splits)
    4 fold records stored    5 fold done, outputs stored

With --fp16 the launches are the uncompressed fp16 decode
(cq_fp16_decode_attn) over the configuration's fp16 K/V, which marks the
same points (3: wave 0's chunks computed).

Each launch is timed from its earliest phase-0 stamp.  The summary gives,
per phase, the median over launches of the median and of the latest
workgroup.  The stamps are issue times: a load or store issued at a phase
completes later.  Launches are eager (one at a time, synchronised), so the
numbers describe one kernel in isolation; bench.py's graph replay overlaps
a launch's start with the previous launch's end.
"""
from __future__ import annotations

import argparse
import os
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
PHASES_LIB = os.path.join(PKG, "libchronoquant_phases.so")

# the workspace carve of cq_decode_common.h: counters, flags, fold records,
# then (m, l) pairs and the partial vectors
_COUNTER_REGION = (64 << 10) + (192 << 10) + 512 * 64 * 12 * 4
NAMES = ["started", "loads issued", "q table ready", "chunk computed", "records stored",
         "fold done"]
TICK_NS = 10.0  # s_memrealtime: 100 MHz


def _round256(x: int) -> int:
    return (x + 255) // 256 * 256


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c1")
    ap.add_argument("--launches", type=int, default=200)
    ap.add_argument("--replicas", type=int, default=57)
    ap.add_argument("--fp16", action="store_true",
                    help="time the uncompressed fp16 decode over the same K/V")
    args = ap.parse_args()
    if not os.path.exists(PHASES_LIB):
        sys.exit(f"{PHASES_LIB} is not built: python -m chronoquant_mlx_amd.build --phases")
    import numpy as np
    import torch

    from chronoquant_mlx_amd import ChronoQuantCache, _lib, synth
    if _lib._lib is not None and _lib.LIB_PATH != PHASES_LIB:
        sys.exit("libchronoquant.so is already loaded in this process")
    _lib.LIB_PATH = PHASES_LIB  # (the package import bound the default path)
    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    k, v = synth.make_kv(cfg)
    kt, vt = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    if args.fp16:
        # replicas so bytes come from HBM
        kvs = [(kt, vt)] + [(kt.clone(), vt.clone()) for _ in range(args.replicas - 1)]
    else:
        base = ChronoQuantCache(stride_k=cfg.stride_k, stride_v=cfg.stride_v,
                                delta_bits_k=cfg.delta_bits_k, delta_bits_v=cfg.delta_bits_v,
                                dead_zone_k=cfg.dead_zone_k, dead_zone_v=cfg.dead_zone_v,
                                capacity=cfg.T)
        base.update_and_fetch(kt, vt)
        import copy
        caches = [base]
        for _ in range(args.replicas - 1):  # cycle replicas so bytes come from HBM
            c = copy.copy(base)
            c._kf = {x: base._kf[x].clone() for x in ("k", "v")}
            c._pk = {x: base._pk[x].clone() for x in ("k", "v")}
            c._sc = {x: base._sc[x].clone() for x in ("k", "v")}
            caches.append(c)
        descs = [c._descriptor() for c in caches]
    q = torch.from_numpy(synth.make_q(cfg)).to(dev)
    out = torch.empty_like(q)
    L = _lib.load()
    B, nq, H = cfg.B, cfg.n_q_heads, cfg.n_kv_heads
    need = L.cq_decode_workspace_size(B, H, nq, cfg.head_dim, cfg.T)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    spans, per_phase = [], []
    nsplit_seen = None
    for i in range(args.launches + 5):
        ws[_COUNTER_REGION:].zero_()
        torch.cuda.synchronize()
        if args.fp16:
            kk, vv = kvs[i % len(kvs)]
            st = L.cq_fp16_decode_attn(kk.data_ptr(), vv.data_ptr(), cfg.T, B, H, cfg.head_dim,
                                       q.data_ptr(), _lib.CQ_F16, nq, cfg.head_dim ** -0.5, None,
                                       cfg.T, cfg.T, out.data_ptr(), _lib.CQ_F16, ws.data_ptr(),
                                       ws.numel(), stream)
        else:
            st = L.cq_decode_attn(descs[i % len(descs)], q.data_ptr(), _lib.CQ_F16, nq,
                                  cfg.head_dim ** -0.5, None, cfg.T, cfg.T, out.data_ptr(),
                                  _lib.CQ_F16, ws.data_ptr(), ws.numel(), stream)
        assert st == 0, _lib.status_string(st)
        torch.cuda.synchronize()
        if i < 5:
            continue  # warm-up
        raw = ws[_COUNTER_REGION:].cpu().numpy()
        found = None
        for ns in range(2, 65):  # the launch's split count (the carve depends on it)
            off = _round256(B * nq * ns * 8)
            n_wg = ns * H * B
            stamps = raw[off: off + n_wg * 64].view(np.uint64).reshape(n_wg, 8)[:, :6]
            if n_wg * 64 <= raw.size - off and np.all(stamps[:, 0] > 0) and \
                    np.all(stamps[:, 5] > 0):
                found = (ns, stamps.astype(np.int64))
                break
        if found is None:
            sys.exit("no phase stamps: the launch did not use the fold records")
        nsplit_seen, stamps = found
        rel = (stamps - stamps[:, 0].min()) * TICK_NS / 1000.0  # us
        spans.append(rel[:, 5].max())
        per_phase.append([(np.median(rel[:, p]), rel[:, p].max()) for p in range(6)])
    pp = np.array(per_phase)  # [launch, phase, (median, max)]
    what = "fp16 decode" if args.fp16 else "config"
    print(f"{what} {args.config}: B={B} H={H} nq={nq} T={cfg.T}; {nsplit_seen} splits per kv head, "
          f"{nsplit_seen * H * B} workgroups; {args.launches} eager launches over "
          f"{args.replicas} cache replicas")
    print(f"{'phase':<18}{'median wg (us)':>16}{'latest wg (us)':>16}")
    for p, name in enumerate(NAMES):
        print(f"{name:<18}{np.median(pp[:, p, 0]):>16.2f}{np.median(pp[:, p, 1]):>16.2f}")
    print(f"first start to last fold: median {np.median(spans):.2f} us "
          f"(p10 {np.percentile(spans, 10):.2f}, p90 {np.percentile(spans, 90):.2f})")


if __name__ == "__main__":
    main()
