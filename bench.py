#!/usr/bin/env python3
"""Benchmark of the fused quantized MoE layer on one MI355X.

Metric: MoE-layer decode tokens/s + achieved HBM GB/s (% of
8 TB/s).  A step is one full layer forward (router GEMV -> top-k -> grouped
w13 + SiLU-gate -> w2 + weighted combine, + the shared expert) over one batch
of synthetic tokens already resident in HBM.  To keep the weights streaming
from HBM rather than the 256 MB last-level cache, ``--layers`` independent
random-init layers (4 x 805 MB for C3) are cycled, one per step, each with a
fresh activation batch -- the pattern a real decode step has across layers.

Prints ONE JSON line.  ``roofline`` covers the dominant kernel (the w13 stage),
timed with HIP events on the launch stream; ``cpu_baseline`` times the
reference's own CPU MoE kernel (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp,
built unmodified into oracle/_ref) on the same routing.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "freetoken-intel_amd"))

METRIC = "MoE-layer decode tokens/s + achieved HBM GB/s (% of 8 TB/s), bs 1-64"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def _parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3_fp8")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--sweep", default="1,4,16,64", help="extra decode batch sizes to report ('' = none)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--offload", action="store_true",
                    help="run the C5 offload decode benchmark instead (64 HBM slots, 256 pinned host banks)")
    ap.add_argument("--offload-steps", type=int, default=200)
    ap.add_argument("--offload-slots", type=int, default=64)
    ap.add_argument("--offload-lru", choices=("device", "host"), default="device",
                    help="C5: LRU planning and copies as GPU kernels (device) or host LRU + per-row memcpy (host)")
    ap.add_argument("--prefill-t", type=int, default=2048,
                    help="prefill chunk measured after the decode points (tiled MFMA stages; 0 = skip)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="measure only the prefill chunk and print its JSON (for counter runs)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the bench, copy a buffer of this many MiB 3 times (a plain copy kernel of known "
                         "size, the reference point for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def _pmc_traffic(kernel: str, config: str, T: int):
    """HBM bytes per launch of the w13 kernel from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the factor the
    same counters read for a copy kernel of known size), if one exists for
    this kernel and workload."""
    path = os.path.join(ROOT, "profiles", f"{kernel}__{config}_T{T}__pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return {"bytes": int(line.split(":", 1)[1].strip()), "source": os.path.relpath(path, ROOT)}
    except OSError:
        pass
    return None


def _w13_bytes_per_expert(syn) -> int:
    return sum(t[0].numel() * t.element_size() for k, t in syn.bank.items() if k.endswith("gate_up")) + (
        syn.bias13[0].numel() * 2 if syn.bias13 is not None else 0)


def main() -> int:
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(expert-parallel sharding is a design note), so --gpus must be 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from ftmoe import _native as nat
    from ftmoe import synthetic as S

    if args.offload:
        return _offload_bench(args)

    dev = torch.device("cuda:0")
    cfg = S.CONFIGS[args.config]
    T = args.batch
    NL = max(1, args.layers)
    NX = 7
    layers, syns = [], []
    for s in range(NL):
        syn = S.generate(cfg, T=T, seed=s, device=dev)
        syns.append(syn)
        layers.append(S.build_layer(syn))
    torch.cuda.synchronize()
    if args.prefill_only:
        print(json.dumps(_prefill_point(cfg, layers, max(1, args.prefill_t), max(4, min(args.steps, 20)))), flush=True)
        return 0
    gx = torch.Generator(device=dev).manual_seed(1234)
    max_t = max([T] + [int(b) for b in args.sweep.split(",") if b])
    x_pool = [torch.randn(max_t, cfg.H, generator=gx, device=dev).to(torch.bfloat16) for _ in range(NX)]

    cap_stream = torch.cuda.Stream(device=dev)

    def graphs_for(xs):
        """One HIP graph per (layer, batch) pair of the rotation: a serving loop
        replays a captured layer forward instead of paying Python launch cost."""
        pairs = [(l, j) for l in range(NL) for j in range(NX)]
        cap_stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cap_stream):
            for l, j in pairs:  # allocates this stream's workspace outside capture
                layers[l].forward(xs[j])
        torch.cuda.current_stream(dev).wait_stream(cap_stream)
        torch.cuda.synchronize()
        gs = {}
        for l, j in pairs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap_stream):
                o = layers[l].forward(xs[j])
            gs[(l, j)] = (g, o)
        # replays must equal the eager forward bit for bit (deterministic kernels)
        ok = True
        for (l, j), (g, o) in list(gs.items())[:3]:
            g.replay()
            ref = layers[l].forward(xs[j])
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(o, ref))
        return gs, ok

    def run_point(Tb: int, steps: int, warmup: int):
        xs = [x[:Tb].contiguous() for x in x_pool]
        for i in range(warmup):
            layers[i % NL].forward(xs[i % NX])
        torch.cuda.synchronize()
        # host wall clock: enqueue + execution, the GPU idle at the start
        w0 = time.perf_counter()
        for i in range(steps):
            j = warmup + i
            layers[j % NL].forward(xs[j % NX])
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - w0) * 1e3 / steps
        # device time: a short sleep kernel queued first lets the host enqueue
        # ahead, so the events see the forwards back to back on the GPU (at
        # T <= 2 a forward's host enqueue, ~20 us of Python and ctypes, is as
        # long as its kernels and would otherwise leave gaps between them); a
        # few untimed forwards after it bring the clocks back up (a 40 ms sleep
        # cost 3-7 % at T >= 16)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if hasattr(torch.cuda, "_sleep"):
            torch.cuda._sleep(2_000_000)
        for i in range(3):
            layers[i % NL].forward(xs[i % NX])
        e0.record()
        for i in range(steps):
            j = warmup + i
            layers[j % NL].forward(xs[j % NX])
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        # the same steps as HIP-graph replays (one captured forward per pair)
        gs, graph_ok = graphs_for(xs)
        for i in range(warmup):
            gs[(i % NL, i % NX)][0].replay()
        torch.cuda.synchronize()
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record()
        for i in range(steps):
            j = warmup + i
            gs[(j % NL, j % NX)][0].replay()
        f1.record()
        torch.cuda.synchronize()
        graph_ms = f0.elapsed_time(f1) / steps
        del gs
        # routing of the same (layer, batch) pairs, untimed: realised unique experts
        uniq = []
        for i in range(steps):
            j = warmup + i
            _, ids, _, _ = layers[j % NL].forward(xs[j % NX], return_routing=True)
            uniq.append(int(torch.unique(ids).numel()))
        b_alg = float(np.mean([S.algorithmic_bytes(cfg, u, Tb) for u in uniq]))
        return ms, wall_ms, float(np.mean(uniq)), b_alg, xs, graph_ms, graph_ok

    ms, wall_ms, U, b_alg, xs, graph_ms, graph_ok = run_point(T, args.steps, args.warmup)
    gbs = b_alg / (ms * 1e-3) / 1e9

    # ---- per-kernel durations.  Each of the five launches of a forward is
    # timed as a group of NL consecutive launches, one per rotated layer (each
    # layer with its own workspace, so the groups keep every layer's stage
    # order), between two events on the launch stream; a sleep kernel queued
    # first lets the host run ahead, so no host gap falls inside a group.
    out = torch.empty(T, cfg.H, dtype=torch.bfloat16, device=dev)
    nsteps = max(1, min(args.steps, 60) // NL)
    stages = (nat.STAGE_ROUTER, nat.STAGE_TOPK, nat.STAGE_W13, nat.STAGE_W2, nat.STAGE_COMBINE)
    wss = [torch.zeros(layers[l].workspace_bytes(T), dtype=torch.uint8, device=dev) for l in range(NL)]
    for st in stages:
        for l in range(NL):
            layers[l].forward_stage(xs[l % NX], out, st, ws=wss[l])
    torch.cuda.synchronize()
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(100_000_000)
    evs = []
    for i in range(nsteps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
        for k, st in enumerate(stages):
            ev[k].record()
            for l in range(NL):
                layers[l].forward_stage(xs[(i + l) % NX], out, st, ws=wss[l])
        ev[-1].record()
        evs.append((ev, i))
    torch.cuda.synchronize()
    kern_us = {name: float(np.mean([ev[k].elapsed_time(ev[k + 1]) for ev, _ in evs])) * 1e3 / NL
               for k, name in enumerate(("router", "topk", "w13", "w2", "combine"))}
    w13_unit = _w13_bytes_per_expert(syns[0])
    sh_w13 = 2 * cfg.shared_inter * cfg.H * 2 if cfg.shared_inter else 0
    bytes_a = []
    for _, i in evs:
        for l in range(NL):
            _, ids, _, _ = layers[l].forward(xs[(i + l) % NX], return_routing=True)
            u = int(torch.unique(ids).numel())
            bytes_a.append(u * w13_unit + sh_w13 + T * cfg.H * 2)
    ach = float(np.mean(bytes_a)) / (kern_us["w13"] * 1e-6) / 1e9
    w13_kernel = layers[0].stage_kernel(T, nat.STAGE_W13)
    traffic = _pmc_traffic(w13_kernel, cfg.name, T)
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic["bytes"] if traffic else None,
                "kernel": f"{w13_kernel} ({cfg.fmt} w13 + activation)",
                "kernel_avg_us": round(kern_us["w13"], 2),
                "bytes_per_launch": int(np.mean(bytes_a)),
                "unit_bytes": w13_unit, "units_per_launch": round((np.mean(bytes_a) - sh_w13 - T * cfg.H * 2) / w13_unit, 2),
                "traffic_source": traffic["source"] if traffic else None,
                "kernels_us": {k: round(v, 2) for k, v in kern_us.items()}}

    # ---- extra decode batch sizes (same layers)
    sweep = []
    for tb in [int(b) for b in args.sweep.split(",") if b]:
        ms_b, wall_b, U_b, balg_b, _, graph_b, _ = run_point(tb, 50, 10)
        g_b = balg_b / (ms_b * 1e-3) / 1e9
        sweep.append({"T": tb, "tokens_per_s": round(tb / (ms_b * 1e-3), 1), "us_per_layer": round(ms_b * 1e3, 2),
                      "wall_us_per_layer": round(wall_b * 1e3, 2), "graph_us_per_layer": round(graph_b * 1e3, 2),
                      "unique_experts": round(U_b, 1), "GBps": round(g_b, 1), "hbm_frac": round(g_b / HBM_PEAK_GBS, 4)})

    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    prefill = _prefill_point(cfg, layers, args.prefill_t, 20) if args.prefill_t > 0 else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(cfg, syns[0], layers[0], xs[0], T, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "wall_ms_per_step": round(wall_ms, 5),
        "graph_ms_per_step": round(graph_ms, 5),
        "timing": "events around K layer forwards launched back to back from Python (one ctypes call each), "
                  "queued behind a sleep kernel so the host runs ahead; wall = host clock around the same K "
                  "forwards without the head start; graph = the same steps as HIP-graph replays (checked "
                  "bitwise against eager: %s)" % ("ok" if graph_ok else "MISMATCH"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "weights": cfg.fmt,
        "data": "synthetic (seeded random-init weights at the real layer shape, N(0,1) bf16 tokens)",
        "config": {"workload": f"{cfg.name} decode T={T}: {cfg.fmt} H={cfg.H} I={cfg.I} E={cfg.E} top-{cfg.k}"
                               + (f" + shared bf16 I={cfg.shared_inter}" if cfg.shared_inter else ""),
                   "global_batch": T, "seq_len": 1, "parallelism": "none (1 GPU)", "layers_rotated": NL},
        "GBps": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "unique_experts": round(U, 2),
        "bytes_per_step": int(b_alg),
        "roofline": roofline,
        "prefill": prefill,
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)
    return 0


def _prefill_point(cfg, layers, T: int, steps: int) -> dict:
    """One prefill chunk of T tokens through the rotated layers: layer time
    (events around back-to-back forwards), per-stage times (each stage of the
    rotation launched as a group, as for decode) and the expert GEMM stages'
    rate against the dense bf16 MFMA peak (the tiles run bf16 MFMAs on weights
    decoded exactly from their quantized form).  FLOPs count real rows only:
    2 * pairs * (2I * H + H * I) routed + the same over T rows for the shared
    expert; padding rows of partly filled tiles are not counted."""
    import numpy as np
    import torch

    from ftmoe import _native as nat

    dev = torch.device("cuda:0")
    NL = len(layers)
    g = torch.Generator(device=dev).manual_seed(4321)
    xs = [torch.randn(T, cfg.H, generator=g, device=dev).to(torch.bfloat16) for _ in range(NL)]
    for i in range(2 * NL):
        layers[i % NL].forward(xs[i % NL])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        layers[i % NL].forward(xs[i % NL])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    out = torch.empty(T, cfg.H, dtype=torch.bfloat16, device=dev)
    stages = (nat.STAGE_ROUTER, nat.STAGE_TOPK, nat.STAGE_W13, nat.STAGE_W2, nat.STAGE_COMBINE)
    wss = [torch.zeros(layers[l].workspace_bytes(T), dtype=torch.uint8, device=dev) for l in range(NL)]
    for st in stages:
        for l in range(NL):
            layers[l].forward_stage(xs[l], out, st, ws=wss[l])
    torch.cuda.synchronize()
    reps = max(1, steps // NL)
    evs = []
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
        for kq, st in enumerate(stages):
            ev[kq].record()
            for l in range(NL):
                layers[l].forward_stage(xs[l], out, st, ws=wss[l])
        ev[-1].record()
        evs.append(ev)
    torch.cuda.synchronize()
    names = ("router", "topk", "w13", "w2", "combine")
    kern = {n: float(np.mean([ev[kq].elapsed_time(ev[kq + 1]) for ev in evs])) * 1e3 / NL for kq, n in enumerate(names)}
    pairs = T * cfg.k
    f13 = 2.0 * pairs * 2 * cfg.I * cfg.H + (2.0 * T * 2 * cfg.shared_inter * cfg.H if cfg.shared_inter else 0.0)
    f2 = 2.0 * pairs * cfg.H * cfg.I + (2.0 * T * cfg.H * cfg.shared_inter if cfg.shared_inter else 0.0)
    tf = (f13 + f2) / ((kern["w13"] + kern["w2"]) * 1e-6) / 1e12
    return {"T": T, "us_per_layer": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
            "kernels_us": {n: round(v, 1) for n, v in kern.items()},
            "kernels": {n: layers[0].stage_kernel(T, st) for n, st in zip(names, stages)},
            "gemm_gflop": round((f13 + f2) / 1e9, 1), "gemm_tflops": round(tf, 1),
            "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
            "w13_tflops": round(f13 / (kern["w13"] * 1e-6) / 1e12, 1),
            "w2_tflops": round(f2 / (kern["w2"] * 1e-6) / 1e12, 1)}


def _zipf_routing(rng, steps: int, T: int, E: int, k: int, s_exp: float = 1.1):
    """Per token k distinct experts drawn Zipf(s) over ranks mapped through a
    seeded permutation; router weights = softmax of N(0, 1) logits over the k."""
    import numpy as np

    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** s_exp
    p /= p.sum()
    ids = np.empty((steps, T, k), np.int32)
    for st in range(steps):
        for t in range(T):
            ids[st, t] = perm[rng.choice(E, k, replace=False, p=p)]
    z = rng.randn(steps, T, k)
    w = np.exp(z - z.max(-1, keepdims=True))
    return ids, (w / w.sum(-1, keepdims=True)).astype(np.float32)


def _offload_bench(args) -> int:
    """C5: the C3 FP8 layer with only ``--offload-slots`` expert slots in HBM and
    all 256 banks in pinned host memory.  Each step: LRU -> copies of the misses
    -> grouped layer call over the slot pool (+ shared expert).  ``device``: the
    LRU and the copies are GPU kernels reading the routing and the pinned banks
    directly (no host synchronisation inside the timed loop); ``host``: the
    host LRU and per-row copies on a side stream.  Reports tokens/s, the hit
    rate over unique expert requests and the achieved H2D GB/s next to a pinned
    256 MiB host-to-device copy."""
    import numpy as np
    import torch

    from ftmoe import synthetic as S
    from ftmoe.moe.offload_cache import OffloadMoeCache, moe_offload_forward

    dev = torch.device("cuda:0")
    cfg = S.CONFIGS["c3_fp8"]
    T, steps, slots = args.batch, args.offload_steps, args.offload_slots
    syn = S.generate(cfg, T=T, seed=0, device=dev)
    bank_host = {k: v.cpu() for k, v in syn.bank.items()}
    del syn.bank
    torch.cuda.empty_cache()
    dev_lru = args.offload_lru == "device"
    cache = OffloadMoeCache(1, cfg.E, slots, dev, quant_format="fp8_block", decode_only=slots < cfg.E,
                            device_lru=dev_lru)
    cache.set_bank_sources({b: [bank_host[b]] for b in cache.bank_schema})
    del bank_host
    rng = np.random.RandomState(0)
    ids_all, w_all = _zipf_routing(rng, steps + 10, T, cfg.E, cfg.k)
    ids_dev = torch.from_numpy(ids_all).to(dev)
    w_dev = torch.from_numpy(w_all).to(dev)
    gx = torch.Generator(device=dev).manual_seed(1234)
    xs = [torch.randn(T, cfg.H, generator=gx, device=dev).to(torch.bfloat16) for _ in range(7)]
    slot_bytes = sum(cache.bank_caches[b][0].numel() * cache.bank_caches[b].element_size() for b in cache.bank_schema)

    def step(i):
        # steps routing to more experts than slots run in chunks that fit the pool
        moe_offload_forward(xs[i % 7], ids_dev[i], w_dev[i], cache, 0, intermediate=cfg.I, shared=syn.shared,
                            ids_host=None if dev_lru else torch.from_numpy(ids_all[i]))

    for i in range(10):  # warm the pool and the kernels
        step(steps + i)
    torch.cuda.synchronize()
    cache.reset_stats()
    uniq = [len(np.unique(ids_all[i])) for i in range(steps)]
    over = sum(u > slots for u in uniq)
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    misses = int(cache.stat_missing)  # counted by the LRU (on the device with device_lru)
    cache.check_status()
    req = int(np.sum(uniq))
    h2d = misses * slot_bytes

    # the achievable pinned H2D rate on this box
    src = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    peak = 5 * (256 << 20) / (e0.elapsed_time(e1) * 1e-3) / 1e9

    line = {
        "metric": "offload decode tokens/s (C5: C3 FP8 layer, 64 HBM slots, 256 pinned host banks)",
        "value": round(steps * T / el, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": 10,
        "ms_per_step": round(el * 1e3 / steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "weights": cfg.fmt,
        "data": "synthetic (seeded random-init FP8 banks at the C3 shape; Zipf(1.1) routing over a seeded "
                "expert permutation, softmax weights of N(0,1) logits)",
        "config": {"workload": f"c5 offload: {cfg.name} T={T}, slots={slots} of E={cfg.E}, one layer",
                   "global_batch": T, "seq_len": 1, "parallelism": "none (1 GPU)"},
        "hit_rate": round(1.0 - misses / req, 4), "misses_per_step": round(misses / steps, 2),
        "unique_experts_per_step": round(float(np.mean(uniq)), 2), "steps_with_more_experts_than_slots": over,
        "h2d_bytes_per_slot": slot_bytes, "h2d_GBps": round(h2d / el / 1e9, 2),
        "h2d_pinned_copy_peak_GBps": round(peak, 2),
        "h2d_frac_of_copy_peak": round(h2d / el / 1e9 / peak, 4),
        "lru": args.offload_lru,
        "timing": ("wall clock around the steps (LRU + copy kernels + layer kernels, enqueued without a host "
                   "synchronisation), synchronised at both ends" if dev_lru else
                   "wall clock around the steps (host LRU + side-stream copies + kernels), synchronised at both ends"),
    }
    print(json.dumps(line), flush=True)
    return 0


def _cpu_baseline(cfg, syn, layer, x, T, seconds):
    """The reference's CPU MoE (cpu_moe.cpp freetoken_cpu_moe_forward_fast) on the
    same layer: banks dequantized to fp32 once outside the timer (by the GPU dequant
    kernel), routing taken from the GPU run, the shared expert as one more
    always-routed expert weighted by its sigmoid gate."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ftm_oracle as O
    from ftmoe.kernel._dequant import dequant

    out, ids, w, _ = layer.forward(x, return_routing=True)
    ids = ids.cpu().numpy()
    w = w.cpu().numpy()
    gu = torch.empty(cfg.E + 1, 2 * cfg.I, cfg.H, dtype=torch.float32)
    dn = torch.empty(cfg.E + 1, cfg.H, cfg.I, dtype=torch.float32)
    for e in range(cfg.E):
        gu[e] = dequant(layer.w13, out_dtype=torch.float32, slot=e).cpu()
        dn[e] = dequant(layer.w2, out_dtype=torch.float32, slot=e).cpu()
    E_tot = cfg.E
    if cfg.shared_inter:
        assert cfg.shared_inter == cfg.I
        gu[cfg.E] = syn.shared["w13"].float().cpu()
        dn[cfg.E] = syn.shared["w2"].float().cpu()
        sl = (x.float() @ syn.shared["gate"].float().T).cpu().numpy()[:, 0]
        sw = O.round_bf16(1.0 / (1.0 + np.exp(-sl)).astype(np.float32))
        ids = np.concatenate([ids, np.full((T, 1), cfg.E, np.int32)], axis=1)
        w = np.concatenate([w, sw[:, None]], axis=1)
        E_tot += 1
    gu_np = gu[:E_tot].numpy()
    dn_np = dn[:E_tot].numpy()
    xf = x.float().cpu().numpy()
    threads = min(16, os.cpu_count() or 1)
    kind = "reference" if O.ref_cpu_moe_available() else "port"

    def call():
        if kind == "reference":
            return O.ref_cpu_moe_forward_fast(xf, ids, w, gu_np, dn_np, threads=threads)
        spec_w13 = O.OracleProj("fp32", gu_np, 2 * cfg.I, cfg.H)
        spec_w2 = O.OracleProj("fp32", dn_np, cfg.H, cfg.I)
        return O.moe_experts(spec_w13, spec_w2, xf, ids, w, E=E_tot, h_bf16=False)

    call()
    n, t0 = 0, time.perf_counter()
    while True:
        call()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(T * n / el, 2), "unit": "tokens/s", "cores": threads if kind == "reference" else 1,
            "kind": kind,
            "sample": f"{n} calls x {T} tokens of {cfg.name} in {el:.1f} s on {model or 'host CPU'}: "
                      "freetoken_cpu_moe_forward_fast (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp, built "
                      "unmodified), fp32 banks dequantized once outside the timer, routing from the GPU run, "
                      "shared expert as an always-routed expert; router GEMV not timed"}


if __name__ == "__main__":
    sys.exit(main())
