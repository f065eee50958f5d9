#!/usr/bin/env python3
"""Benchmark of the fused quantized MoE layer on one MI355X.

Metric: MoE-layer decode tokens/s + achieved HBM GB/s (% of
8 TB/s), bs 1-64.  A step is one full layer forward (router GEMV -> top-k ->
grouped w13 + gate activation -> w2 + weighted combine, + the shared expert)
over one batch of synthetic tokens already resident in HBM.  The weights
stream from HBM, not the 256 MB last-level cache: ``--layers`` independent
random-init layers of each config are cycled, one per step (4 x 805 MB for
C3), each step with a fresh activation batch, as a real decode step has
across layers.

Every BASELINE config is measured in the one JSON line the driver reads:

* ``value`` / ``ms_per_step``: the headline, C3 FP8 (256 experts, top-8 +
  shared expert) decode at T=16 -- ``configs[2]`` of BASELINE.json;
* ``configs``: C1 INT8 T=4; C2 GPTQ T=1/4/16/64; C3 T=1..64 and the
  2048-token prefill chunk; C4 MXFP4 T=1/32/128 and the 4096-token prefill;
  C5 offload (64 HBM slots, 256 pinned host banks, 200 Zipf steps).  Each
  decode point: tokens/s, GB/s and fraction of 8 TB/s from the median over
  batches of 10 back-to-back forwards, ``--steps`` forwards in all (mean
  beside it);
  each config's w13 and w2 kernels against the HBM roofline (stage events on
  the launch stream); prefill: the GEMM stages against the dense bf16 MFMA
  peak;
* ``cpu_baseline``: the reference's own CPU MoE kernel
  (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp, built unmodified into
  oracle/_ref) on the same routing, on the host cores of the GPU box, for
  every config: all cores clamped to E (the kernel's own rule,
  cpu_moe.cpp:485-490), one thread, and "reference-equivalent" with the
  per-call full-bank fp32 conversion of python/freetoken/kernel/cpu_moe.py:460-461.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "freetoken-intel_amd"))

METRIC = "MoE-layer decode tokens/s + achieved HBM GB/s (% of 8 TB/s), bs 1-64"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
HEADLINE = ("c3_fp8", 16)
# decode batches and the dominant-kernel point of each config
DECODE_T = {"c1_int8": (4,), "c2_gptq": (1, 4, 16, 64), "c3_fp8": (1, 2, 4, 8, 16, 32, 64),
            "c4_mxfp4": (1, 32, 128)}
KERNEL_T = {"c1_int8": 4, "c2_gptq": 16, "c3_fp8": 16, "c4_mxfp4": 32}


def _parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed forwards per decode point")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="c1_int8,c2_gptq,c3_fp8,c4_mxfp4,c5",
                    help="comma list of configs to measure (c5 = the offload decode)")
    ap.add_argument("--point", default="",
                    help="measure only one decode point, CONFIG:T (for profiler runs; no CPU baseline)")
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU work per baseline row")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", default="", help="measure only this config's prefill chunk (counter runs)")
    ap.add_argument("--offload-steps", type=int, default=200)
    ap.add_argument("--offload-slots", type=int, default=64)
    ap.add_argument("--offload-lru", choices=("device", "host"), default="device",
                    help="C5: LRU planning and copies as GPU kernels (device) or host LRU + per-row memcpy (host)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the bench, copy a buffer of this many MiB 3 times (a plain copy kernel of known "
                         "size, the reference point for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# ------------------------------------------------------------------ helpers
def _pmc_traffic(kernel: str, config: str, T: int):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the factor the same
    counters read for a copy kernel of known size), if one exists for this
    kernel and workload."""
    path = os.path.join(ROOT, "profiles", f"{kernel}__{config}_T{T}__pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return {"bytes": int(line.split(":", 1)[1].strip()), "source": os.path.relpath(path, ROOT)}
    except OSError:
        pass
    return None


def _proj_bytes(syn, which: str) -> int:
    """Bytes of one routed expert's projection ``which`` (gate_up / down) incl. its bias."""
    n = sum(t[0].numel() * t.element_size() for k, t in syn.bank.items() if k.endswith(which))
    bias = syn.bias13 if which == "gate_up" else syn.bias2
    return n + (bias[0].numel() * 2 if bias is not None else 0)


def _cpu_info() -> dict:
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)", "CPU family",
                       "Model", "Hypervisor vendor", "L3 cache"):
                info[key] = val
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        info["cpus_available_to_process"] = len(os.sched_getaffinity(0))
    except OSError:
        pass
    return info


def _median(v):
    import numpy as np

    return float(np.median(np.asarray(v, np.float64)))


# ------------------------------------------------------------------ decode
class ConfigBench:
    """NL rotated random-init layers of one config on the GPU."""

    def __init__(self, cfg, NL: int, max_t: int):
        import torch

        from ftmoe import synthetic as S

        self.cfg = cfg
        self.dev = torch.device("cuda:0")
        self.syns, self.layers = [], []
        for s in range(NL):
            syn = S.generate(cfg, T=1, seed=s, device=self.dev)
            self.syns.append(syn)
            self.layers.append(S.build_layer(syn))
        gx = torch.Generator(device=self.dev).manual_seed(1234)
        self.NX = 7
        self.x_pool = [torch.randn(max_t, cfg.H, generator=gx, device=self.dev).to(torch.bfloat16)
                       for _ in range(self.NX)]
        torch.cuda.synchronize()

    def xs(self, T):
        return [x[:T].contiguous() for x in self.x_pool]

    def decode_point(self, T: int, steps: int, warmup: int, graphs: bool = False, batch: int = 10) -> dict:
        """Layer time over ``steps`` forwards of T tokens: the median over
        batches of ``batch`` back-to-back forwards, each batch between two HIP
        events on the launch stream (queued behind a short sleep kernel so the
        host runs ahead and the events see GPU time only), and the mean over
        all of them; the rotation's realised unique experts and B_alg.  An
        event marker serialises the kernels on either side of it (about 2.7 us
        at C3 T=16), so markers go between batches, not between forwards."""
        import numpy as np
        import torch

        from ftmoe import synthetic as S

        NL, NX = len(self.layers), self.NX
        xs = self.xs(T)
        for i in range(warmup):
            self.layers[i % NL].forward(xs[i % NX])
        torch.cuda.synchronize()
        # host wall clock: enqueue + execution
        w0 = time.perf_counter()
        for i in range(steps):
            self.layers[(warmup + i) % NL].forward(xs[(warmup + i) % NX])
        torch.cuda.synchronize()
        wall_us = (time.perf_counter() - w0) * 1e6 / steps
        # device time: events every `batch` forwards
        nb = max(1, steps // batch)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(nb + 1)]
        if hasattr(torch.cuda, "_sleep"):
            torch.cuda._sleep(2_000_000)
        for i in range(3):  # clocks back up after the sleep
            self.layers[i % NL].forward(xs[i % NX])
        for b in range(nb):
            ev[b].record()
            for i in range(batch):
                j = warmup + b * batch + i
                self.layers[j % NL].forward(xs[j % NX])
        ev[nb].record()
        torch.cuda.synchronize()
        per = [ev[b].elapsed_time(ev[b + 1]) * 1e3 / batch for b in range(nb)]
        uniq = []
        for i in range(min(steps, 4 * NL * NX)):
            j = warmup + i
            _, ids, _, _ = self.layers[j % NL].forward(xs[j % NX], return_routing=True)
            uniq.append(int(torch.unique(ids).numel()))
        b_alg = float(np.mean([S.algorithmic_bytes(self.cfg, u, T) for u in uniq]))
        med = _median(per)
        res = {"T": T, "us_per_layer": round(med, 2), "us_mean": round(float(np.mean(per)), 2),
               "timed_forwards": nb * batch, "wall_us_per_layer": round(wall_us, 2),
               "tokens_per_s": round(T / (med * 1e-6), 1), "unique_experts": round(float(np.mean(uniq)), 2),
               "bytes": int(b_alg), "GBps": round(b_alg / (med * 1e-6) / 1e9, 1),
               "hbm_frac": round(b_alg / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if graphs:
            g = self._graph_point(xs, steps, warmup)
            res["graph_us_per_layer"], res["graph_bitwise_equal"] = g["step"], g["bitwise_equal"]
            res["graph_step_layers"] = g["layers"]
            res["graph1_us_per_layer"] = g["single"]
        return res

    def _graph_point(self, xs, steps, warmup, step_layers: int = 48):
        """HIP-graph replays, as an engine uses them (``MoeGraphRunner``: one
        graph per decode step): a step of ``step_layers`` forwards (the rotated
        layers and inputs in turn) captured in one graph and replayed, us per
        layer; beside it one captured forward per (layer, input) pair replayed
        in turn (``single``), which pays a graph launch per forward.  Outputs
        are checked bitwise against eager forwards."""
        import torch

        NL, NX = len(self.layers), self.NX
        cap = torch.cuda.Stream(device=self.dev)
        pairs = [(l, j) for l in range(NL) for j in range(NX)]
        cap.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(cap):
            for l, j in pairs:  # sizes this stream's workspace outside capture
                self.layers[l].forward(xs[j])
        torch.cuda.current_stream(self.dev).wait_stream(cap)
        torch.cuda.synchronize()

        def timed(fn, reps):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            f0.record()
            for _ in range(reps):
                fn()
            f1.record()
            torch.cuda.synchronize()
            return f0.elapsed_time(f1) * 1e3 / reps

        seq = [(i % NL, i % NX) for i in range(step_layers)]
        gstep = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gstep, stream=cap):
            outs = [self.layers[l].forward(xs[j]) for l, j in seq]
        ok = True
        gstep.replay()
        for (l, j), o in list(zip(seq, outs))[-3:]:
            ref = self.layers[l].forward(xs[j])
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(o, ref))
        step_us = timed(gstep.replay, max(1, steps // step_layers)) / step_layers
        gs = {}
        for l, j in pairs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                o = self.layers[l].forward(xs[j])
            gs[(l, j)] = (g, o)
        for (l, j), (g, o) in list(gs.items())[:3]:
            g.replay()
            ref = self.layers[l].forward(xs[j])
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(o, ref))
        order = [gs[((warmup + i) % NL, (warmup + i) % NX)][0] for i in range(steps)]
        it = iter(range(10 ** 9))

        def one():
            order[next(it) % len(order)].replay()

        single_us = timed(one, steps)
        return {"step": round(step_us, 2), "layers": step_layers, "single": round(single_us, 2),
                "bitwise_equal": ok}

    def stage_times(self, T: int, reps: int = 15, passes: int = 4) -> dict:
        """Average duration of each of the five stage launches at T tokens: each
        stage is launched as a group of `passes` x NL consecutive launches, the
        rotated layers in turn (each layer with its own workspace, so the groups
        keep every layer's stage order; a stage launched again on its workspace
        recomputes the same outputs), between two events on the launch stream,
        so the cost of each group boundary (the event, the first launch's ramp)
        is spread over passes x NL launches; a sleep kernel queued first lets
        the host run ahead."""
        import numpy as np
        import torch

        from ftmoe import _native as nat

        NL, NX = len(self.layers), self.NX
        xs = self.xs(T)
        out = torch.empty(T, self.cfg.H, dtype=torch.bfloat16, device=self.dev)
        stages = (nat.STAGE_ROUTER, nat.STAGE_TOPK, nat.STAGE_W13, nat.STAGE_W2, nat.STAGE_COMBINE)
        wss = [torch.zeros(self.layers[l].workspace_bytes(T), dtype=torch.uint8, device=self.dev) for l in range(NL)]
        for st in stages:
            for l in range(NL):
                self.layers[l].forward_stage(xs[l % NX], out, st, ws=wss[l])
        torch.cuda.synchronize()
        if hasattr(torch.cuda, "_sleep"):
            torch.cuda._sleep(100_000_000)
        evs = []
        for i in range(reps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
            for k, st in enumerate(stages):
                ev[k].record()
                for _ in range(passes):
                    for l in range(NL):
                        self.layers[l].forward_stage(xs[(i + l) % NX], out, st, ws=wss[l])
            ev[-1].record()
            evs.append((ev, i))
        torch.cuda.synchronize()
        us = {name: float(np.mean([ev[k].elapsed_time(ev[k + 1]) for ev, _ in evs])) * 1e3 / (NL * passes)
              for k, name in enumerate(("router", "topk", "w13", "w2", "combine"))}
        # realised unique experts of the same (layer, batch) pairs
        uniq = []
        for _, i in evs:
            for l in range(NL):
                _, ids, _, _ = self.layers[l].forward(xs[(i + l) % NX], return_routing=True)
                uniq.append(int(torch.unique(ids).numel()))
        return {"us": us, "unique": float(np.mean(uniq)), "xs": xs}

    def rooflines(self, T: int) -> dict:
        """The w13 and w2 kernels at T tokens against the HBM roofline:
        algorithmic bytes per launch (realised unique experts x the projection's
        bytes per expert + the shared expert's projection + activations) over
        the kernel's average launch duration."""
        from ftmoe import _native as nat

        st = self.stage_times(T)
        cfg, syn, U = self.cfg, self.syns[0], st["unique"]
        us = st["us"]
        Is = cfg.shared_inter
        out = {"kernels_us": {k: round(v, 2) for k, v in us.items()}, "unique_experts": round(U, 2)}
        for stage, which, name, sh_bytes, act_bytes in (
                ("w13", "gate_up", nat.STAGE_W13, 2 * Is * cfg.H * 2, T * cfg.H * 2),
                ("w2", "down", nat.STAGE_W2, cfg.H * Is * 2, T * (cfg.k + (1 if Is else 0)) * cfg.I * 2)):
            unit = _proj_bytes(syn, which)
            b = U * unit + sh_bytes + act_bytes
            kern = self.layers[0].stage_kernel(T, name)
            ach = b / (us[stage] * 1e-6) / 1e9
            traffic = _pmc_traffic(kern, cfg.name, T)
            out[stage] = {"bound": "hbm", "kernel": kern, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                          "traffic": traffic["bytes"] if traffic else None,
                          "traffic_source": traffic["source"] if traffic else None,
                          "kernel_avg_us": round(us[stage], 2), "bytes_per_launch": int(b), "unit_bytes": unit,
                          "units_per_launch": round(U, 2)}
        return out

    def prefill_point(self, T: int, steps: int = 12) -> dict:
        """One prefill chunk of T tokens through the rotated layers: layer time
        (events around back-to-back forwards), per-stage times and the expert
        GEMM stages' rate against the dense bf16 MFMA peak (the tiles run bf16
        MFMAs on weights decoded exactly from their quantized form).  FLOPs
        count real rows only: 2 * pairs * (2I * H + H * I) routed + the same
        over T rows for the shared expert; padding rows of partly filled tiles
        are not counted."""
        import numpy as np
        import torch

        from ftmoe import _native as nat

        cfg, dev = self.cfg, self.dev
        NL = len(self.layers)
        g = torch.Generator(device=dev).manual_seed(4321)
        xs = [torch.randn(T, cfg.H, generator=g, device=dev).to(torch.bfloat16) for _ in range(NL)]
        for i in range(2 * NL):
            self.layers[i % NL].forward(xs[i % NL])
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        for i in range(steps):
            ev[i].record()
            self.layers[i % NL].forward(xs[i % NL])
        ev[steps].record()
        torch.cuda.synchronize()
        us = _median([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(steps)])
        out = torch.empty(T, cfg.H, dtype=torch.bfloat16, device=dev)
        stages = (nat.STAGE_ROUTER, nat.STAGE_TOPK, nat.STAGE_W13, nat.STAGE_W2, nat.STAGE_COMBINE)
        wss = [torch.zeros(self.layers[l].workspace_bytes(T), dtype=torch.uint8, device=dev) for l in range(NL)]
        for st in stages:
            for l in range(NL):
                self.layers[l].forward_stage(xs[l], out, st, ws=wss[l])
        torch.cuda.synchronize()
        evs = []
        for _ in range(max(1, steps // NL)):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
            for kq, st in enumerate(stages):
                e[kq].record()
                for l in range(NL):
                    self.layers[l].forward_stage(xs[l], out, st, ws=wss[l])
            e[-1].record()
            evs.append(e)
        torch.cuda.synchronize()
        names = ("router", "topk", "w13", "w2", "combine")
        kern = {n: float(np.mean([e[kq].elapsed_time(e[kq + 1]) for e in evs])) * 1e3 / NL
                for kq, n in enumerate(names)}
        pairs = T * cfg.k
        Is = cfg.shared_inter
        f13 = 2.0 * pairs * 2 * cfg.I * cfg.H + 2.0 * T * 2 * Is * cfg.H
        f2 = 2.0 * pairs * cfg.H * cfg.I + 2.0 * T * cfg.H * Is
        tf = (f13 + f2) / ((kern["w13"] + kern["w2"]) * 1e-6) / 1e12
        syn = self.syns[0]
        w_bytes = cfg.E * (_proj_bytes(syn, "gate_up") + _proj_bytes(syn, "down")) + cfg.E * cfg.H * 2 + 3 * cfg.H * Is * 2
        b_alg = w_bytes + 2 * T * cfg.H * 2
        return {"T": T, "us_per_layer": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
                "GBps": round(b_alg / (us * 1e-6) / 1e9, 1),
                "hbm_frac": round(b_alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "kernels_us": {n: round(v, 1) for n, v in kern.items()},
                "kernels": {n: self.layers[0].stage_kernel(T, st) for n, st in zip(names, stages)},
                "gemm_gflop": round((f13 + f2) / 1e9, 1), "gemm_tflops": round(tf, 1),
                "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                "w13_tflops": round(f13 / (kern["w13"] * 1e-6) / 1e12, 1),
                "w2_tflops": round(f2 / (kern["w2"] * 1e-6) / 1e12, 1)}


# ------------------------------------------------------------------ CPU baseline
def _cpu_baselines(cb: ConfigBench, T: int, seconds: float) -> dict:
    """The reference's CPU MoE (cpu_moe.cpp freetoken_cpu_moe_forward_fast) on
    the config's layer and the GPU run's routing at T tokens, three rows:

    * ``all_cores``: threads = 0, the kernel's own rule (hardware concurrency
      clamped to E, cpu_moe.cpp:485-490), fp32 banks dequantized once outside
      the timer (by the GPU dequant kernel);
    * ``one_thread``: the same, threads = 1;
    * ``reference_equivalent``: what python/freetoken/kernel/cpu_moe.py:460-461
      does per call: the dense bf16 banks converted to fp32 (whole [E,2I,H] and
      [E,H,I]) inside the timer, then the all-cores call.

    The shared expert (C3) rides as one more always-routed expert weighted by
    its sigmoid gate; the router GEMV is not timed.  Each row runs calls for
    about ``seconds`` (at least one)."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ftm_oracle as O
    from ftmoe.kernel._dequant import dequant

    if not O.ref_cpu_moe_available():
        return {"rows": [], "note": "oracle/_ref/libcpu_moe_ref.so not built"}
    cfg, layer, syn = cb.cfg, cb.layers[0], cb.syns[0]
    x = cb.x_pool[0][:T].contiguous()
    _, ids, w, _ = layer.forward(x, return_routing=True)
    ids, w = ids.cpu().numpy(), w.cpu().numpy()
    E_tot = cfg.E + (1 if cfg.shared_inter else 0)
    Imax = max(cfg.I, cfg.shared_inter)
    assert not cfg.shared_inter or cfg.shared_inter == cfg.I
    gu_bf = torch.empty(E_tot, 2 * cfg.I, cfg.H, dtype=torch.bfloat16)
    dn_bf = torch.empty(E_tot, cfg.H, Imax, dtype=torch.bfloat16)
    gu = torch.empty(E_tot, 2 * cfg.I, cfg.H, dtype=torch.float32)
    dn = torch.empty(E_tot, cfg.H, Imax, dtype=torch.float32)
    for e in range(cfg.E):
        a = dequant(layer.w13, out_dtype=torch.float32, slot=e)
        b = dequant(layer.w2, out_dtype=torch.float32, slot=e)
        gu[e], dn[e] = a.cpu(), b.cpu()
        gu_bf[e], dn_bf[e] = a.to(torch.bfloat16).cpu(), b.to(torch.bfloat16).cpu()
    if cfg.shared_inter:
        gu[cfg.E], dn[cfg.E] = syn.shared["w13"].float().cpu(), syn.shared["w2"].float().cpu()
        gu_bf[cfg.E], dn_bf[cfg.E] = syn.shared["w13"].cpu(), syn.shared["w2"].cpu()
        sl = (x.float() @ syn.shared["gate"].float().T).cpu().numpy()[:, 0]
        sw = O.round_bf16((1.0 / (1.0 + np.exp(-sl))).astype(np.float32))
        ids = np.concatenate([ids, np.full((T, 1), cfg.E, np.int32)], axis=1)
        w = np.concatenate([w, sw[:, None]], axis=1)
    gu_np, dn_np = gu.numpy(), dn.numpy()
    xf = x.float().cpu().numpy()

    def timed(fn):
        fn()  # warm (page-in, thread start-up)
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return n, el

    def ref_equiv():
        a, b = gu_bf.to(torch.float32).contiguous(), dn_bf.to(torch.float32).contiguous()
        return O.ref_cpu_moe_forward_fast(xf, ids, w, a.numpy(), b.numpy(), threads=0)

    rows = []
    hw = os.cpu_count() or 1
    for name, fn, threads in (("all_cores", lambda: O.ref_cpu_moe_forward_fast(xf, ids, w, gu_np, dn_np, threads=0),
                               min(hw, E_tot)),
                              ("one_thread", lambda: O.ref_cpu_moe_forward_fast(xf, ids, w, gu_np, dn_np, threads=1), 1),
                              ("reference_equivalent", ref_equiv, min(hw, E_tot))):
        n, el = timed(fn)
        tps = T * n / el
        b_alg = _alg_bytes_fp32(cfg, ids, T)
        rows.append({"row": name, "tokens_per_s": round(tps, 2), "ms_per_call": round(el * 1e3 / n, 3),
                     "threads": threads, "calls": n, "seconds": round(el, 2),
                     "GBps_fp32_banks": round(b_alg * n / el / 1e9, 2)})
    return {"T": T, "rows": rows}


def _alg_bytes_fp32(cfg, ids, T):
    """Bytes the CPU kernel streams per call: the fp32 rows of every expert it
    touches (realised unique experts incl. the shared one) + x and out."""
    import numpy as np

    u = len(np.unique(ids))
    Imax = max(cfg.I, cfg.shared_inter)
    return u * (2 * cfg.I * cfg.H + cfg.H * Imax) * 4 + 2 * T * cfg.H * 4


# ------------------------------------------------------------------ C5 offload
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


def _offload_bench(args) -> dict:
    """C5: the C3 FP8 layer with only ``--offload-slots`` expert slots in HBM and
    all 256 banks in pinned host memory.  Each step: LRU -> copies of the
    misses -> grouped layer call over the slot pool (+ shared expert).
    ``device``: the LRU and the copies are GPU kernels reading the routing and
    the pinned banks directly (no host synchronisation inside the timed loop);
    ``host``: the host LRU and per-row copies on a side stream.  Reports
    tokens/s, the hit rate over unique expert requests and the achieved H2D
    GB/s next to a pinned 256 MiB host-to-device copy."""
    import numpy as np
    import torch

    from ftmoe import synthetic as S
    from ftmoe.moe.offload_cache import OffloadMoeCache, moe_offload_forward

    dev = torch.device("cuda:0")
    cfg = S.CONFIGS["c3_fp8"]
    T, steps, slots = 16, args.offload_steps, args.offload_slots
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
    del cache
    torch.cuda.empty_cache()
    return {
        "workload": f"c5 offload: c3_fp8 T={T}, slots={slots} of E={cfg.E}, one layer, {steps} Zipf(1.1) steps",
        "tokens_per_s": round(steps * T / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
        "hit_rate": round(1.0 - misses / req, 4), "misses_per_step": round(misses / steps, 2),
        "unique_experts_per_step": round(float(np.mean(uniq)), 2), "steps_with_more_experts_than_slots": over,
        "h2d_bytes_per_slot": slot_bytes, "h2d_GBps": round(h2d / el / 1e9, 2),
        "h2d_pinned_copy_peak_GBps": round(peak, 2),
        "roofline": {"bound": "pcie_h2d", "achieved": round(h2d / el / 1e9, 2), "peak": round(peak, 2),
                     "unit": "GB/s", "frac": round(h2d / el / 1e9 / peak, 4),
                     "peak_source": "5 x 256 MiB pinned host-to-device copies on this box"},
        "lru": args.offload_lru,
        "timing": ("wall clock around the steps (LRU + copy kernels + layer kernels, enqueued without a host "
                   "synchronisation), synchronised at both ends" if dev_lru else
                   "wall clock around the steps (host LRU + side-stream copies + kernels), synchronised at both "
                   "ends"),
    }


# ------------------------------------------------------------------ main
def _config_line(cb: ConfigBench, args, T_list, with_cpu: bool) -> dict:
    import torch

    cfg = cb.cfg
    res = {"name": cfg.name, "workload": f"{cfg.fmt} H={cfg.H} I={cfg.I} E={cfg.E} top-{cfg.k}"
                                        + (f" + shared bf16 I={cfg.shared_inter}" if cfg.shared_inter else ""),
           "decode": []}
    for T in T_list:
        res["decode"].append(cb.decode_point(T, args.steps, args.warmup, graphs=(cfg.name, T) == HEADLINE))
        torch.cuda.synchronize()
    kt = KERNEL_T[cfg.name]
    if kt in T_list:
        res["kernel_T"] = kt
        res["rooflines"] = cb.rooflines(kt)
    if cfg.prefill and not args.no_prefill:
        res["prefill"] = cb.prefill_point(cfg.prefill)
    if with_cpu:
        res["cpu_baseline"] = _cpu_baselines(cb, kt, args.cpu_seconds)
    return res


def main() -> int:
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(expert-parallel sharding is a design note), so --gpus must be 1.", file=sys.stderr)
        return 2

    import torch

    from ftmoe import synthetic as S

    if args.prefill_only:
        cfg = S.CONFIGS[args.prefill_only]
        cb = ConfigBench(cfg, max(1, args.layers), 1)
        print(json.dumps(cb.prefill_point(cfg.prefill)), flush=True)
        return 0
    if args.point:
        name, T = args.point.split(":")
        cfg = S.CONFIGS[name]
        cb = ConfigBench(cfg, max(1, args.layers), int(T))
        line = {"point": args.point, "decode": cb.decode_point(int(T), args.steps, args.warmup),
                "rooflines": cb.rooflines(int(T))}
        if args.copy_probe_mib > 0:
            _copy_probe(args.copy_probe_mib)
        print(json.dumps(line), flush=True)
        return 0

    want = [c.strip() for c in args.configs.split(",") if c.strip()]
    configs = {}
    t_start = time.perf_counter()
    for name in ("c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"):
        if name not in want:
            continue
        cfg = S.CONFIGS[name]
        T_list = DECODE_T[name]
        cb = ConfigBench(cfg, max(1, args.layers), max(T_list))
        configs[name] = _config_line(cb, args, T_list, with_cpu=not args.no_cpu_baseline)
        del cb
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    if "c5" in want:
        configs["c5_offload"] = _offload_bench(args)
    if args.copy_probe_mib > 0:
        _copy_probe(args.copy_probe_mib)

    c3 = configs.get(HEADLINE[0])
    head = next((d for d in c3["decode"] if d["T"] == HEADLINE[1]), None) if c3 else None
    cpu_info = _cpu_info()
    cpu = None
    if c3 and "cpu_baseline" in c3 and c3["cpu_baseline"].get("rows"):
        r = next(r for r in c3["cpu_baseline"]["rows"] if r["row"] == "all_cores")
        cpu = {"value": r["tokens_per_s"], "unit": "tokens/s", "cores": r["threads"], "kind": "reference",
               "sample": f"{r['calls']} calls x {HEADLINE[1]} tokens of c3_fp8 in {r['seconds']} s: "
                         "freetoken_cpu_moe_forward_fast (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp, "
                         "built unmodified), threads=0 (all cores clamped to E), fp32 banks dequantized once "
                         "outside the timer, routing from the GPU run, shared expert as an always-routed "
                         "expert, router GEMV not timed; one-thread and reference-equivalent rows per config "
                         "under configs.*.cpu_baseline",
               "host": cpu_info}
    roof = None
    if c3 and "rooflines" in c3:
        r13 = c3["rooflines"]["w13"]
        roof = dict(r13)
        roof["kernel"] = f"{r13['kernel']} (fp8_block w13 + activation, C3 T={HEADLINE[1]})"
        roof["kernels_us"] = c3["rooflines"]["kernels_us"]
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"] if head else None,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_layer"] * 1e-3, 5) if head else None,
        "ms_per_step_mean": round(head["us_mean"] * 1e-3, 5) if head else None,
        "timing": f"median over {args.steps // 10} batches of 10 back-to-back layer forwards ({args.steps} timed), "
                  "HIP events on the launch stream between batches, forwards queued behind a sleep kernel so the "
                  "host runs ahead; mean, host wall clock and HIP-graph replay beside it; weights rotated over "
                  f"{args.layers} random-init layers per config so they stream from HBM",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "weights": "fp8_block",
        "data": "synthetic (seeded random-init weights at the real layer shapes, N(0,1) bf16 tokens)",
        "config": {"workload": f"c3_fp8 decode T={HEADLINE[1]}: fp8_block H=2048 I=512 E=256 top-8 + shared bf16 "
                               "I=512 (BASELINE.json configs[2]); every other config under 'configs'",
                   "global_batch": HEADLINE[1], "seq_len": 1, "parallelism": "none (1 GPU)",
                   "layers_rotated": args.layers},
        "GBps": head["GBps"] if head else None,
        "hbm_frac": head["hbm_frac"] if head else None,
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": configs,
        "bench_seconds": round(time.perf_counter() - t_start, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


def _copy_probe(mib: int) -> None:
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


if __name__ == "__main__":
    sys.exit(main())
