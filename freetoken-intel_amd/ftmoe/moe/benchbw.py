"""Calibrate the hybrid split on this machine: the host CPU expert GEMV against
the PCIe gather into the GPU slot pool, per expert format, and write the
per-GPU profile :mod:`ftmoe.moe.bench_profile` reads (the ``ft bench bw``
command, python/freetoken/moe/benchbw.py:1-535).

Per format, on one layer of ``E`` experts at the model's ``(H, I)``:

* **CPU GEMV** -- ``ftm_cpu_moe_forward`` (the hybrid backend's CPU half)
  for one decode token routed to all ``E`` experts, reading the packed host
  banks, on every core up to ``E`` threads.  Bytes = ``E`` x the packed
  bytes of one expert (weights + scales / zeros / biases).
* **PCIe gather** -- the offload half itself: ``OffloadMoeCache.ensure_experts``
  + ``copy_missing`` of all ``E`` experts from pinned host banks into the
  slot pool (a two-layer pool alternating layers, so every step misses every
  expert).  Same bytes.
* **Overlapped** -- both at once, the CPU half on its own thread (the ctypes
  call releases the interpreter lock), each half's bytes over its own time
  while the other runs (benchbw.py:243-326 divides both by one shared wall
  time; see :func:`bench_overlap`).
* **HBM** (reported, not used by the split) -- a device-to-device copy of the
  same bytes.

Verdict (benchbw.py:329-348): ``hybrid`` when the standalone CPU bandwidth is
above ``HYBRID_CPU_OVER_PCIE_THRESHOLD`` x the PCIe one, else ``offload``; the
fetch fraction ``pcie / (pcie + cpu)`` of the overlapped pair (standalone
pair if the overlap run failed).

Where the reference counts ``3 I H`` elements at a nominal width per format
(benchbw.py:86-131, 1 byte for fp8 without its scales) and uses dense
fp32/bf16 banks for the CPU half whatever the format, here the banks are the
format's own packed banks and the bytes are theirs, so every format's CPU
figure is the one the hybrid step will see.  The profile's device block is
``"gpu": {"name", "uuid"}``.

Run: ``python -m ftmoe.moe.benchbw [--dtype fp8_block,gptq_int4 | all]
[--model PATH] [--experts E --intermediate I --hidden H] [--out PATH]``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import threading
import time
from typing import Optional

HYBRID_CPU_OVER_PCIE_THRESHOLD = 2.0

# the bare command's shape: Qwen3-30B-A3B-like (H 2048, I 768, 64 experts), bf16
_DEFAULT_NUM_EXPERTS = 64
_DEFAULT_MOE_INTERMEDIATE = 768
_DEFAULT_HIDDEN = 2048
_DEFAULT_DTYPE = "bf16"

_WARMUP_ITERS = 3
_MEASURE_ITERS = 10

FORMATS = ("bf16", "fp8_block", "gptq_int4", "int8_channel", "mxfp4")
_GROUP = {"fp8_block": 128, "gptq_int4": 128, "mxfp4": 32}
# checkpoint quant_method -> format (ftmoe.loader.load_moe_expert_sources)
_METHOD_TO_FORMAT = {"gptq": "gptq_int4", "fp8": "fp8_block", "mxfp4": "mxfp4", "compressed-tensors": "int8_channel"}


def synthetic_banks(fmt: str, E: int, intermediate: int, hidden: int, *, distinct: int = 4, seed: int = 0,
                    bias: bool = False) -> dict:
    """``{bank name: [E, ...] host tensor}`` of ``fmt`` for ``E`` experts: ``distinct``
    experts drawn N(0, 0.02) and quantized, repeated to ``E`` rows (separate
    memory, so every expert is its own read); ``bias`` adds MXFP4 expert biases."""
    import torch

    from ..synthetic import quantize_bank

    if fmt not in FORMATS:
        raise ValueError(f"unknown expert format {fmt!r} (one of {FORMATS})")
    d = max(1, min(distinct, E))
    g = torch.Generator().manual_seed(seed)
    grp = _GROUP.get(fmt, 128)
    bank = quantize_bank(fmt, torch.randn(d, 2 * intermediate, hidden, generator=g) * 0.02, "gate_up", group=grp)
    bank.update(quantize_bank(fmt, torch.randn(d, hidden, intermediate, generator=g) * 0.02, "down", group=grp))
    if bias and fmt == "mxfp4":
        bank["bias_gate_up"] = (torch.randn(d, 2 * intermediate, generator=g) * 0.02).to(torch.bfloat16)
        bank["bias_down"] = (torch.randn(d, hidden, generator=g) * 0.02).to(torch.bfloat16)
    reps = -(-E // d)
    return {k: v.repeat(reps, *([1] * (v.dim() - 1)))[:E].contiguous() for k, v in bank.items()}


def expert_bytes(bank: dict) -> int:
    """Packed bytes of one expert across every bank."""
    return sum(t[0].numel() * t.element_size() for t in bank.values())


def _cpu_layer(fmt: str, bank: dict, E: int, intermediate: int, hidden: int):
    from .hybrid import host_layer_from_bank

    return host_layer_from_bank(fmt, bank, num_experts=E, intermediate=intermediate, topk=E,
                                group=_GROUP.get(fmt), int8_k=(hidden, intermediate),
                                bias13=bank.get("bias_gate_up"), bias2=bank.get("bias_down"))


class _CpuHalf:
    """One decode token routed to all ``E`` experts on the host CPU kernel."""

    def __init__(self, fmt: str, bank: dict, E: int, intermediate: int, hidden: int, threads: int = 0) -> None:
        import torch

        self.layer, self._keep = _cpu_layer(fmt, bank, E, intermediate, hidden)
        self.x = torch.randn(1, hidden)
        self.ids = torch.arange(E, dtype=torch.int32).reshape(1, E)
        self.w = torch.full((1, E), 1.0 / E)
        self.out = torch.empty(1, hidden)
        self.threads = threads

    def run(self) -> None:
        import ctypes

        from .. import _native as nat

        rc = nat.lib().ftm_cpu_moe_forward(ctypes.byref(self.layer), self.x.data_ptr(), 1, self.ids.data_ptr(),
                                           self.w.data_ptr(), None, int(self.threads), 0, self.out.data_ptr())
        nat.check(rc, "ftm_cpu_moe_forward")


class _PcieHalf:
    """Every step PCIe-fetches all ``E`` experts into the slot pool: a two-layer
    pool of ``E`` slots whose steps alternate layers."""

    def __init__(self, fmt: str, bank: dict, E: int, intermediate: int, hidden: int, device) -> None:
        import torch

        from .offload_cache import OffloadMoeCache

        self.cache = OffloadMoeCache(2, E, E, device, quant_format=fmt)
        self.cache.set_bank_sources({b: [t, t] for b, t in bank.items()})
        self.ids = torch.arange(E)
        self.i = 0

    def run(self) -> None:
        self.cache.ensure_experts(self.i % 2, self.ids)
        self.cache.copy_missing()
        self.i += 1


def _timed(fn, iters: int, sync=None) -> float:
    for _ in range(_WARMUP_ITERS):
        fn()
    if sync:
        sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    if sync:
        sync()
    return time.perf_counter() - t0


def bench_cpu_moe(fmt: str, bank: dict, E: int, intermediate: int, hidden: int, *, iters: Optional[int] = None,
                  threads: int = 0) -> float:
    """Host CPU expert GEMV bandwidth, GB/s (benchbw.py:194-240).  Needs no GPU."""
    iters = iters or _MEASURE_ITERS
    half = _CpuHalf(fmt, bank, E, intermediate, hidden, threads)
    secs = _timed(half.run, iters)
    return E * expert_bytes(bank) * iters / 1e9 / secs


def bench_pcie_gather(fmt: str, bank: dict, E: int, intermediate: int, hidden: int, device, *,
                      iters: Optional[int] = None) -> float:
    """Slot-pool PCIe gather bandwidth, GB/s (benchbw.py:134-191), wall clock
    around the offload half's own calls."""
    import torch

    iters = iters or _MEASURE_ITERS
    half = _PcieHalf(fmt, bank, E, intermediate, hidden, device)
    secs = _timed(half.run, iters, lambda: torch.cuda.synchronize(device))
    return E * expert_bytes(bank) * iters / 1e9 / secs


def bench_hbm_copy(nbytes: int, device, *, iters: Optional[int] = None) -> float:
    """Device-to-device copy bandwidth over ``nbytes``, GB/s (read + write)."""
    import torch

    iters = iters or _MEASURE_ITERS
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    secs = _timed(lambda: dst.copy_(src), iters, lambda: torch.cuda.synchronize(device))
    return 2 * nbytes * iters / 1e9 / secs


def bench_overlap(fmt: str, bank: dict, E: int, intermediate: int, hidden: int, device, *,
                  iters: Optional[int] = None, threads: int = 0) -> tuple:
    """``(pcie_gbs, cpu_gbs)`` with both halves running at once: the CPU half
    loops on a host thread while this thread issues gathers (each waited for,
    as a decode step waits for its copies), and each half keeps going until
    both have done ``iters`` steps, so neither runs uncontended.  Each half's
    rate is its own steps' bytes over its own time.

    The reference (benchbw.py:243-326) divides both halves' bytes by the one
    shared wall time, which makes the two overlapped figures equal whenever the
    byte counts are (every format there), so its fetch fraction is always 0.5;
    the per-half rates here are what the bandwidth-matched split needs."""
    import torch

    iters = iters or _MEASURE_ITERS
    cpu = _CpuHalf(fmt, bank, E, intermediate, hidden, threads)
    pcie = _PcieHalf(fmt, bank, E, intermediate, hidden, device)
    for _ in range(_WARMUP_ITERS):
        cpu.run()
        pcie.run()
    torch.cuda.synchronize(device)
    n_cpu, n_pcie = [0], [0]
    t_cpu, err = [0.0], []

    def cpu_loop():
        try:
            while n_cpu[0] < iters or n_pcie[0] < iters:
                cpu.run()
                n_cpu[0] += 1
                t_cpu[0] = time.perf_counter()
        except Exception as exc:  # reported after the join
            err.append(exc)

    th = threading.Thread(target=cpu_loop, daemon=True)
    t0 = time.perf_counter()
    th.start()
    t_pcie = t0
    while (n_pcie[0] < iters or n_cpu[0] < iters) and not err:
        pcie.run()
        torch.cuda.synchronize(device)
        n_pcie[0] += 1
        t_pcie = time.perf_counter()
    th.join()
    if err:
        raise err[0]
    b = E * expert_bytes(bank) / 1e9
    return b * n_pcie[0] / (t_pcie - t0), b * n_cpu[0] / (t_cpu[0] - t0)


def _recommend(pcie_gbs: Optional[float], cpu_gbs: Optional[float]) -> str:
    """``hybrid`` iff the CPU bandwidth beats the PCIe one by the threshold (benchbw.py:329-333)."""
    if pcie_gbs is None or cpu_gbs is None or pcie_gbs <= 0:
        return "offload"
    return "hybrid" if cpu_gbs > HYBRID_CPU_OVER_PCIE_THRESHOLD * pcie_gbs else "offload"


def _fetch_fraction(pcie_ov, cpu_ov, pcie, cpu) -> float:
    """``pcie / (pcie + cpu)``, overlapped pair first (benchbw.py:336-348)."""
    if pcie_ov and cpu_ov:
        return min(1.0, pcie_ov / (pcie_ov + cpu_ov))
    if pcie and cpu:
        return min(1.0, pcie / (pcie + cpu))
    return 0.0


def bench_format(device, fmt: str, E: int, intermediate: int, hidden: int, *, iters: Optional[int] = None,
                 threads: int = 0, bias: bool = False) -> dict:
    """One format's profile entry (benchbw.py:351-367)."""
    bank = synthetic_banks(fmt, E, intermediate, hidden, bias=bias)
    per = expert_bytes(bank)
    cpu = bench_cpu_moe(fmt, bank, E, intermediate, hidden, iters=iters, threads=threads)
    pcie = bench_pcie_gather(fmt, bank, E, intermediate, hidden, device, iters=iters)
    pcie_ov, cpu_ov = bench_overlap(fmt, bank, E, intermediate, hidden, device, iters=iters, threads=threads)
    hbm = bench_hbm_copy(E * per, device, iters=iters)
    frac = _fetch_fraction(pcie_ov, cpu_ov, pcie, cpu)
    return {"cpu_moe_gbs": round(cpu, 3), "pcie_gather_gbs": round(pcie, 3),
            "cpu_moe_overlap_gbs": round(cpu_ov, 3), "pcie_gather_overlap_gbs": round(pcie_ov, 3),
            "hbm_copy_gbs": round(hbm, 3), "recommended": _recommend(pcie, cpu),
            "fetch_fraction": round(frac, 4) if frac else None, "bytes_per_expert": per, "experts": E,
            "cpu_threads": threads or min(E, os.cpu_count() or 1)}


def model_shapes(model_path: str) -> tuple:
    """``(E, I, H, [format])`` of a checkpoint's ``config.json`` (the reference's
    ``_model_shapes``, benchbw.py:370-405); the format from its quantization
    (unquantized -> bf16)."""
    from ..loader import checkpoint_is_int8_pack_quantized, checkpoint_quant_method, moe_checkpoint_config

    c = moe_checkpoint_config(model_path)
    method = checkpoint_quant_method(model_path)
    if method is None:
        fmt = "bf16"
    elif method == "compressed-tensors" and not checkpoint_is_int8_pack_quantized(model_path):
        raise ValueError(f"{model_path!r}: compressed-tensors checkpoint that is not int8 pack-quantized")
    else:
        fmt = _METHOD_TO_FORMAT.get(method)
        if fmt is None:
            raise ValueError(f"{model_path!r}: quantization {method!r} has no expert bank in this build")
    return c.num_experts, c.moe_intermediate_size, c.hidden_size, [fmt]


def parse_argv(argv=None, prog: str = "ft bench bw") -> argparse.Namespace:
    """The reference's flags (benchbw.py:408-462), ``--dtype`` also taking a
    comma list or ``all``, plus ``--threads`` for the CPU half."""
    p = argparse.ArgumentParser(prog=prog, description=(
        "Calibrate the host CPU expert GEMV against the PCIe gather into the GPU slot pool and pick the MoE "
        "backend (hybrid/offload) and the hybrid fetch fraction; writes a per-GPU profile JSON."))
    p.add_argument("--dtype", default=None, help="expert format(s): " + ", ".join(FORMATS) + ", comma list or all")
    p.add_argument("--model", default=None, help="checkpoint directory: its E / I / H and format")
    p.add_argument("--experts", type=int, default=None)
    p.add_argument("--intermediate", type=int, default=None)
    p.add_argument("--hidden", type=int, default=None)
    p.add_argument("--out", default=None, help="profile path (default: per-GPU file under $XDG_CACHE_HOME)")
    p.add_argument("--repeats", type=int, default=None, help=f"measured iterations (default {_MEASURE_ITERS})")
    p.add_argument("--threads", type=int, default=0, help="CPU half threads (0 = every core, at most E)")
    p.add_argument("--quiet", action="store_true", help="print only the profile JSON")
    return p.parse_args(sys.argv[1:] if argv is None else argv)


def resolve_workload(args: argparse.Namespace) -> tuple:
    """``(E, I, H, formats)`` from the defaults, ``--model`` and the overrides."""
    from .bench_profile import quant_format_for_dtype

    E, I, H, fmts = _DEFAULT_NUM_EXPERTS, _DEFAULT_MOE_INTERMEDIATE, _DEFAULT_HIDDEN, [_DEFAULT_DTYPE]
    if args.model:
        E, I, H, fmts = model_shapes(args.model)
    E = args.experts or E
    I = args.intermediate or I
    H = args.hidden or H
    if args.dtype:
        fmts = list(FORMATS) if args.dtype == "all" else [quant_format_for_dtype(d.strip())
                                                          for d in args.dtype.split(",") if d.strip()]
    bad = [f for f in fmts if f not in FORMATS]
    if bad:
        raise ValueError(f"unknown expert format(s) {bad} (one of {FORMATS})")
    return E, I, H, fmts


def main(argv=None, prog: str = "ft bench bw") -> int:
    """Measure every requested format and write the profile (benchbw.py:465-532).
    No GPU: an error and exit code 1 (the profile is device-specific)."""
    from .bench_profile import default_profile_path, gpu_identity, is_gpu_available

    args = parse_argv(argv, prog)
    if not is_gpu_available():
        print(f"{prog}: needs a ROCm GPU (none visible)", file=sys.stderr)
        return 1
    import torch

    E, I, H, fmts = resolve_workload(args)
    iters = args.repeats if args.repeats and args.repeats > 0 else _MEASURE_ITERS
    name, uuid = gpu_identity()
    out = args.out or default_profile_path(uuid)
    os.makedirs(os.path.dirname(out) or ".", exist_ok=True)
    device = torch.device("cuda", 0)
    profile = {"gpu": {"name": name, "uuid": uuid}, "dtypes": {}, "dtype_kernels": {},
               "generated_at": time.strftime("%Y-%m-%d %H:%M:%S %Z"),
               "threshold_cpu_over_pcie": HYBRID_CPU_OVER_PCIE_THRESHOLD,
               "shape": {"experts": E, "intermediate": I, "hidden": H}}
    if not args.quiet:
        print(f"{prog}: {name} (uuid {uuid or 'unknown'})  E={E} I={I} H={H}  formats={','.join(fmts)}")
    for fmt in fmts:
        entry = bench_format(device, fmt, E, I, H, iters=iters, threads=args.threads)
        profile["dtypes"][fmt] = entry["recommended"]
        profile["dtype_kernels"][fmt] = entry
        if not args.quiet:
            print(f"  {fmt}: cpu {entry['cpu_moe_gbs']} GB/s  pcie {entry['pcie_gather_gbs']} GB/s  overlapped "
                  f"cpu {entry['cpu_moe_overlap_gbs']} / pcie {entry['pcie_gather_overlap_gbs']} GB/s  "
                  f"hbm {entry['hbm_copy_gbs']} GB/s -> {entry['recommended']}, fetch {entry['fetch_fraction']}")
    with open(out, "w") as f:
        json.dump(profile, f, indent=2)
    if args.quiet:
        print(json.dumps(profile, indent=2))
    else:
        print(f"profile written to {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main(prog="python -m ftmoe.moe.benchbw"))


__all__ = ["main", "parse_argv", "bench_format", "synthetic_banks", "expert_bytes", "model_shapes",
           "HYBRID_CPU_OVER_PCIE_THRESHOLD"]
