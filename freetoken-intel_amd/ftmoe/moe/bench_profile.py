"""Reader of the bandwidth-calibration profile: the offload-family backend and
the hybrid fetch fraction for an expert format on this GPU
(python/freetoken/moe/bench_profile.py:1-301).

``ftmoe.moe.benchbw`` measures, per expert format, the host CPU expert GEMV and
the PCIe gather into the slot pool, alone and overlapped, and writes one JSON
profile per GPU.  This module reads it at start-up -- it imports no torch at
module level, and touches the GPU only to learn its name and UUID when the
caller gives neither -- and

* recommends ``"hybrid"`` when the profile says the CPU GEMV beat the PCIe
  gather by the threshold, else ``"offload"`` (:func:`load_backend_recommendation`);
* yields the hybrid backend's fetch fraction ``f = pcie / (pcie + cpu)`` of the
  overlapped pair (:func:`load_hybrid_fetch_fraction`).

Lookup (the reference's): an explicit ``path``, else ``$FREETOKEN_BENCHBW_PATH``,
else ``$XDG_CACHE_HOME/freetoken/benchbw/<gpu uuid>.json``, else the legacy
``.../freetoken/benchbw.json``.  A profile measured on a differently named
device is ignored (``None``: the caller keeps its default, ``offload``).  The
device block is read from ``"gpu"`` (what ``benchbw`` writes) or ``"xpu"``
(profiles of the reference's Intel port).

Format keys are this build's ``quant_format`` names; the reference's
``"mxfp4_triton"`` key is read as ``"mxfp4"``.  Unlike the reference, whose
CPU half takes dense banks only, every format here has a CPU kernel, so
every format may resolve to ``hybrid``.
"""
from __future__ import annotations

import json
import os
from typing import Any, Optional

# engine quant_format -> profile key (identity here; the CPU half serves every format)
_QUANT_TO_BENCH_FORMAT = {"bf16": "bf16", "fp8_block": "fp8_block", "gptq_int4": "gptq_int4",
                          "int8_channel": "int8_channel", "mxfp4": "mxfp4"}

# CLI / reference spellings -> profile keys
_FORMAT_ALIASES = {"fp8": "fp8_block", "mxfp4_triton": "mxfp4", "gptq": "gptq_int4", "int8": "int8_channel"}

# torch dtype names -> profile keys (bench_profile.py:45-52)
_DTYPES_TO_FORMAT = {"bfloat16": "bf16", "float16": "fp16", "float32": "fp32"}

ENV_PROFILE_PATH = "FREETOKEN_BENCHBW_PATH"


def quant_format_for_dtype(dtype: Any) -> Optional[str]:
    """The profile key for a torch dtype or format spelling, ``None`` when empty
    (bench_profile.py:55-69): ``torch.bfloat16`` -> ``"bf16"``, ``"fp8"`` ->
    ``"fp8_block"``; anything else passes through."""
    if dtype is None:
        return None
    dt = str(dtype).lower()
    if dt.startswith("torch."):
        dt = dt[len("torch."):]
    if not dt:
        return None
    return _FORMAT_ALIASES.get(dt, _DTYPES_TO_FORMAT.get(dt, dt))


def _cache_dir() -> str:
    cache = os.environ.get("XDG_CACHE_HOME") or os.path.expanduser("~/.cache")
    return os.path.join(cache, "freetoken")


def default_profile_path(gpu_uuid: Optional[str] = None) -> str:
    """``$XDG_CACHE_HOME/freetoken/benchbw/<gpu uuid>.json`` -- one file per
    device, bandwidths differ between slots -- else the legacy ``benchbw.json``
    (bench_profile.py:77-85)."""
    if gpu_uuid:
        return os.path.join(_cache_dir(), "benchbw", f"{gpu_uuid}.json")
    return os.path.join(_cache_dir(), "benchbw.json")


def latest_profile_path() -> Optional[str]:
    """The newest ``benchbw/*.json``, else the legacy file, else ``None``
    (bench_profile.py:88-108)."""
    per_gpu = os.path.join(_cache_dir(), "benchbw")
    best = None
    try:
        names = os.listdir(per_gpu)
    except OSError:
        names = []
    for name in names:
        if not name.endswith(".json"):
            continue
        p = os.path.join(per_gpu, name)
        try:
            m = os.path.getmtime(p)
        except OSError:
            continue
        if best is None or m > best[0]:
            best = (m, p)
    if best is not None:
        return best[1]
    legacy = default_profile_path()
    return legacy if os.path.isfile(legacy) else None


def _load(path) -> Optional[dict]:
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def is_gpu_available() -> bool:
    """A ROCm GPU is visible to torch (imported here, not at module level)."""
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available())


def gpu_identity() -> tuple:
    """``(name, uuid)`` of GPU 0, each ``None`` when unknown or no GPU."""
    if not is_gpu_available():
        return None, None
    import torch

    try:
        props = torch.cuda.get_device_properties(0)
    except Exception:
        return None, None
    name = str(getattr(props, "name", "") or "") or None
    uuid = str(getattr(props, "uuid", "") or "") or None
    return name, uuid


# Which calibration profile to trust (the reference's lookup contract,
# bench_profile.py:138-183, restated as rules):
#   1. the sources: an explicit path (argument, else $FREETOKEN_BENCHBW_PATH)
#      is the only source; otherwise this device's file (when its uuid is
#      known), then the legacy single file;
#   2. the first source that exists decides: a JSON object is the profile, any
#      other content (unreadable, not JSON, not an object) means "keep the
#      default" -- later sources are not consulted;
#   3. a profile whose recorded device name differs from the known name of
#      this device is ignored (measurements are hardware-specific);
#   4. the device identity is queried only when the caller gave neither a path
#      nor a name nor a uuid.
# Every outcome is (profile or None, the source that decided or None).


def _profile_sources(path, uuid: Optional[str]) -> tuple:
    explicit = path or os.environ.get(ENV_PROFILE_PATH)
    if explicit:
        return (explicit,)
    return ((default_profile_path(uuid),) if uuid else ()) + (default_profile_path(),)


def _recorded_device_name(prof: dict) -> Optional[str]:
    """The device name a profile was measured on (this build writes ``gpu``,
    the reference ``xpu``)."""
    for key in ("gpu", "xpu"):
        dev = prof.get(key)
        if isinstance(dev, dict) and dev.get("name"):
            return str(dev["name"])
    return None


def _usable_profile(gpu_name: Optional[str], path, gpu_uuid: Optional[str] = None) -> tuple:
    """``(profile, source)`` to trust, or ``(None, source)`` -- see the rules above."""
    if path is None and gpu_name is None and gpu_uuid is None:
        gpu_name, gpu_uuid = gpu_identity()
    decided = next((src for src in _profile_sources(path, gpu_uuid) if os.path.exists(src)), None)
    if decided is None:
        return None, None
    prof = _load(decided)
    if not isinstance(prof, dict):
        return None, decided
    measured_on = _recorded_device_name(prof)
    if gpu_name and measured_on and measured_on != gpu_name:
        return None, decided
    return prof, decided


def _keys(quant_format: str) -> list:
    fmt = quant_format_for_dtype(quant_format) or quant_format
    fmt = _QUANT_TO_BENCH_FORMAT.get(fmt, fmt)
    return [fmt, "mxfp4_triton"] if fmt == "mxfp4" else [fmt]


def _entries(prof: dict, keys: list) -> list:
    """Per-dtype kernel entries first, then every per-model workload's."""
    out = []
    for k in keys:
        out.append((prof.get("dtype_kernels") or {}).get(k))
    for wl in (prof.get("workloads") or {}).values():
        if isinstance(wl, dict):
            for k in keys:
                out.append((wl.get("kernels") or {}).get(k))
    return [e for e in out if isinstance(e, dict)]


def load_backend_recommendation(quant_format: str, gpu_name: Optional[str] = None, path=None,
                                gpu_uuid: Optional[str] = None, *, xpu_name: Optional[str] = None,
                                xpu_uuid: Optional[str] = None) -> Optional[str]:
    """``"hybrid"`` / ``"offload"`` for ``quant_format`` from the profile, or
    ``None`` (no usable profile, no entry) -- bench_profile.py:186-226: the
    per-dtype verdict first; else the per-model workloads sharing the format,
    ``hybrid`` only when all of them say so.  ``xpu_name`` / ``xpu_uuid`` are
    the reference's spellings of ``gpu_name`` / ``gpu_uuid``."""
    prof, _ = _usable_profile(gpu_name or xpu_name, path, gpu_uuid or xpu_uuid)
    if prof is None:
        return None
    keys = _keys(quant_format)
    dtypes = prof.get("dtypes")
    if isinstance(dtypes, dict):
        for k in keys:
            if dtypes.get(k) in ("hybrid", "offload"):
                return dtypes[k]
    workloads = prof.get("workloads")
    if not isinstance(workloads, dict):
        return None
    picks = []
    for wl in workloads.values():
        if not isinstance(wl, dict):
            continue
        for k in keys:
            e = (wl.get("kernels") or {}).get(k)
            if isinstance(e, dict) and e.get("recommended"):
                picks.append(e["recommended"])
    if not picks:
        return None
    return "hybrid" if all(p == "hybrid" for p in picks) else "offload"


def load_hybrid_fetch_fraction(quant_format: str, gpu_name: Optional[str] = None, path=None,
                               gpu_uuid: Optional[str] = None, *, xpu_name: Optional[str] = None,
                               xpu_uuid: Optional[str] = None) -> Optional[float]:
    """The hybrid fetch fraction for ``quant_format``, or ``None``
    (bench_profile.py:229-265): ``pcie_ov / (pcie_ov + cpu_ov)`` of the first
    entry holding the overlapped pair; an entry with only the standalone pair
    gives ``pcie / cpu`` -- the reference reader's fallback formula, pinned by
    its test (tests/test_moe_hybrid_profile.py:194-201: 10 / 30) though its
    writer stores ``pcie / (pcie + cpu)``.  Clamped to at most 1; a zero
    bandwidth gives ``None``."""
    prof, _ = _usable_profile(gpu_name or xpu_name, path, gpu_uuid or xpu_uuid)
    if prof is None:
        return None
    for e in _entries(prof, _keys(quant_format)):
        cpu_ov, pcie_ov = e.get("cpu_moe_overlap_gbs"), e.get("pcie_gather_overlap_gbs")
        if cpu_ov and pcie_ov:
            return min(1.0, pcie_ov / (pcie_ov + cpu_ov))
        cpu, pcie = e.get("cpu_moe_gbs"), e.get("pcie_gather_gbs")
        if cpu and pcie:
            return min(1.0, pcie / cpu)
    return None


def resolve_backend(backend, *, is_moe: bool, quant_format: Optional[str] = None) -> Optional[str]:
    """Resolve ``"auto"`` (bench_profile.py:268-292): an explicit backend passes
    through; a dense model or a box without a GPU gets ``"fused"``; an MoE on a
    GPU gets the profile's recommendation for its format, else ``"offload"``."""
    if backend != "auto":
        return backend
    if not is_moe or not is_gpu_available():
        return "fused"
    if quant_format is not None:
        rec = load_backend_recommendation(quant_format)
        if rec is not None:
            return rec
    return "offload"


__all__ = ["default_profile_path", "latest_profile_path", "load_backend_recommendation", "load_hybrid_fetch_fraction",
           "resolve_backend", "quant_format_for_dtype", "gpu_identity", "ENV_PROFILE_PATH", "_FORMAT_ALIASES"]
