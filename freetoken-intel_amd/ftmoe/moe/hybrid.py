"""Hybrid CPU || GPU split of a decode step's routed experts, every bank format.

The reference's hybrid backend (python/freetoken/models/qwen3_moe/__init__.py:
679-866) partitions a decode step's distinct routed experts: a fraction ``f``
is PCIe-fetched into the device slot pool and computed by the GPU, the rest
is computed by the host CPU from the same pinned host banks, the two halves
run concurrently and their outputs are summed.  ``f`` is the calibrated
bandwidth-matched fetch fraction (``ftmoe.moe.benchbw``).  The reference
CPU kernel takes only dense fp32 / bf16 banks, so quantized checkpoints fall
back to pure offload there (:730-733); here the CPU half is
``ftm_cpu_moe_forward`` (``csrc/ftm_cpu.cpp``), which decodes GPTQ, FP8,
INT8 and MXFP4 banks itself, so the split serves every format.

Split rule, as the reference's: ``n`` distinct routed experts, ``n_fetch =
round(n * f)`` clamped to ``[1, n - 1]`` (and to ``max_fetch``), the CPU
takes the ``n - n_fetch`` lowest expert ids.  The CPU half runs on the
library's worker thread (``ftm_cpu_moe_submit``) while the GPU half --
``moe_offload_forward`` with the CPU's experts passed as ``-1`` -- is
enqueued; the CPU half's fp32 output is copied to the GPU, added in fp32 to
the GPU half's (which its layer call rounded to the activation dtype) and the
sum is rounded to the activation dtype.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _native as nat
from ..banks import proj_from_bank


def host_layer_from_bank(fmt: str, bank: dict, *, num_experts: int, intermediate: int, topk: int,
                         group: Optional[int] = None, int8_k: Optional[tuple] = None, bias13=None, bias2=None,
                         act: str = "silu", swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0):
    """``(ftm_moe_layer, keepalive)`` over HOST expert banks ``{bank name: [E, ...]}``
    (the ``_BANK_SCHEMAS`` names; expert ``e`` = row ``e``), for
    ``ftm_cpu_moe_forward``.  ``int8_k``: the logical ``(K_gate_up, K_down)``."""
    from ..layer import ACTIVATIONS

    if fmt == "bf16":
        H = int(bank["gate_up"].shape[-1])
    elif fmt == "fp8_block":
        H = int(bank["weight_gate_up"].shape[-1])
    elif fmt == "gptq_int4":
        H = int(bank["qweight_gate_up"].shape[1]) * 8
        if group is None:
            raise ValueError("gptq_int4 banks need their group size")
    elif fmt == "int8_channel":
        H = int(int8_k[0])
    elif fmt == "mxfp4":
        H = int(bank["blocks_gate_up"].shape[2]) * 32
    else:
        raise ValueError(f"hybrid CPU half: quant_format {fmt!r} has no CPU kernel")
    kd = int(int8_k[1]) if fmt == "int8_channel" else intermediate
    b13 = bias13.contiguous() if bias13 is not None else None
    b2 = bias2.contiguous() if bias2 is not None else None
    w13 = proj_from_bank(fmt, bank, which="gate_up", N=2 * intermediate, K=H, group=group, bias=b13)
    w2 = proj_from_bank(fmt, bank, which="down", N=H, K=kd, group=group, bias=b2)
    L = nat.FtmMoeLayer()
    L.w13, L.w2 = w13.c(), w2.c()
    L.num_experts = int(num_experts)
    L.hidden, L.inter, L.topk = H, int(intermediate), int(topk)
    L.act = ACTIVATIONS[act]
    L.swiglu_alpha, L.swiglu_limit = float(swiglu_alpha), float(swiglu_limit)
    L.act_dtype = nat.DT_F32
    L.h_dtype = nat.DT_F32
    return L, (w13, w2, bank)


def host_layer(cache, layer_id: int, *, intermediate: int, topk: int, act: str = "silu",
               swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0):
    """The same over one layer's pinned host banks of a slot pool (MXFP4 biases:
    the pool's optional ``bias_gate_up`` / ``bias_down`` banks)."""
    fmt = cache.quant_format
    if fmt == "gptq_int4" and getattr(cache, "gptq_group_size", None) is None:
        raise ValueError("OffloadMoeCache.gptq_group_size is not set (the hybrid CPU half refuses to guess)")
    group = {"gptq_int4": getattr(cache, "gptq_group_size", None), "fp8_block": getattr(cache, "fp8_block_size", 128),
             "mxfp4": 32}.get(fmt)
    src = cache.bank_sources
    b13 = src["bias_gate_up"][layer_id] if "bias_gate_up" in src else None
    b2 = src["bias_down"][layer_id] if "bias_down" in src else None
    int8_k = (cache.int8_k_gate_up, cache.int8_k_down) if fmt == "int8_channel" else None
    return host_layer_from_bank(fmt, {b: src[b][layer_id] for b in cache.bank_schema},
                                num_experts=cache.num_experts, intermediate=intermediate, topk=topk, group=group,
                                int8_k=int8_k, bias13=b13, bias2=b2, act=act, swiglu_alpha=swiglu_alpha,
                                swiglu_limit=swiglu_limit)


def cpu_moe_forward(layer, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                    expert_mask: Optional[torch.Tensor] = None, *, threads: int = 0,
                    force_scalar: bool = False) -> torch.Tensor:
    """``ftm_cpu_moe_forward`` on host tensors: fp32 ``[T, H]`` routed output of
    the experts in ``expert_mask`` (uint8 ``[E]``, None = all)."""
    x = x.to("cpu", torch.float32).contiguous()
    ids = topk_ids.to("cpu", torch.int32).contiguous()
    w = topk_w.to("cpu", torch.float32).contiguous()
    mask = expert_mask.to("cpu", torch.uint8).contiguous() if expert_mask is not None else None
    out = torch.empty(x.shape, dtype=torch.float32)
    rc = nat.lib().ftm_cpu_moe_forward(ctypes.byref(layer), x.data_ptr(), int(x.shape[0]), ids.data_ptr(),
                                       w.data_ptr(), nat.ptr(mask), int(threads), 1 if force_scalar else 0,
                                       out.data_ptr())
    nat.check(rc, "ftm_cpu_moe_forward")
    return out


class CpuJob:
    """A CPU-half call running on the library's worker thread; :meth:`result`
    waits for it (once) and returns its fp32 output.

    The worker holds one job at a time and reads this job's buffers until it
    is waited for, so a job must always be waited for: :meth:`discard` waits
    and drops the output (the error path of a step), and a job that is
    garbage-collected without either is waited for then."""

    def __init__(self, layer, x, ids, w, mask, out, keep) -> None:
        self._keep = (layer, x, ids, w, mask, out, keep)  # alive until the worker is done with them
        self._out = out
        self._rc: Optional[int] = None
        self._done = False
        self._handle = int(nat.lib().ftm_cpu_moe_submit(ctypes.byref(layer), x.data_ptr(), int(x.shape[0]),
                                                        ids.data_ptr(), w.data_ptr(), nat.ptr(mask), 0,
                                                        out.data_ptr()))
        nat.check(self._handle, "ftm_cpu_moe_submit")

    def _wait(self) -> int:
        if self._rc is None:
            self._rc = int(nat.lib().ftm_cpu_moe_wait(self._handle))
        return self._rc

    def result(self) -> torch.Tensor:
        if self._done:
            raise RuntimeError("CpuJob.result() called twice")
        self._done = True
        nat.check(self._wait(), "ftm_cpu_moe_wait")
        return self._out

    def discard(self) -> None:
        """Wait for the job to finish and drop its output."""
        self._wait()
        self._done = True

    def __del__(self) -> None:
        if getattr(self, "_rc", 0) is None and getattr(self, "_handle", -1) > 0:
            try:
                self._wait()
            except Exception:  # interpreter shutdown: the library may already be gone
                pass


def split_experts(ids_host: torch.Tensor, fetch_fraction: float, max_fetch: int = -1) -> Optional[set]:
    """The experts the CPU computes for this step (qwen3_moe/__init__.py:733-752):
    of the ``n`` distinct routed ids, all but ``n_fetch = round(n * f)`` (clamped
    to ``max_fetch`` and to ``[1, n - 1]``), lowest ids first.  None = no split
    (``f`` outside ``(0, 1)`` or fewer than two experts)."""
    if not 0.0 < fetch_fraction < 1.0:
        return None
    seen = sorted({int(e) for e in ids_host.reshape(-1).tolist() if int(e) >= 0})
    n = len(seen)
    if n < 2:
        return None
    n_fetch = int(round(n * fetch_fraction))
    if 0 <= max_fetch < n_fetch:
        n_fetch = max_fetch
    n_fetch = max(1, min(n - 1, n_fetch))
    return set(seen[: n - n_fetch])


def moe_hybrid_forward(flat: torch.Tensor, top_idx: torch.Tensor, top_w: torch.Tensor, cache, layer_id: int, *,
                       intermediate: int, fetch_fraction: float, max_fetch: int = -1, act: str = "silu",
                       shared: Optional[dict] = None, swiglu_alpha: float = 1.702,
                       swiglu_limit: float = 7.0) -> torch.Tensor:
    """One decode step of the routed experts (+ shared expert on the GPU) split
    between the CPU and the GPU (see the module docstring).  Falls back to the
    pure offload step when there is nothing to split."""
    from .offload_cache import moe_offload_forward

    ids_host = top_idx.to("cpu", torch.int32)
    cpu_experts = split_experts(ids_host, fetch_fraction, max_fetch)
    kw = dict(intermediate=intermediate, act=act, shared=shared, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)
    if not cpu_experts:
        return moe_offload_forward(flat, top_idx, top_w, cache, layer_id, ids_host=ids_host.to(torch.int64), **kw)
    E = cache.num_experts
    mask = torch.zeros(E, dtype=torch.uint8)
    mask[sorted(cpu_experts)] = 1
    layer, keep = host_layer(cache, layer_id, intermediate=intermediate, topk=int(top_idx.shape[1]), act=act,
                             swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)
    x_h = flat.to("cpu", torch.float32).contiguous()
    w_h = top_w.to("cpu", torch.float32).contiguous()
    out_h = torch.empty(x_h.shape, dtype=torch.float32, pin_memory=flat.is_cuda)
    job = CpuJob(layer, x_h, ids_host.contiguous(), w_h, mask, out_h, keep)
    try:
        # the GPU half: the same routing with the CPU's experts as pairs without an expert
        on_cpu = mask.to(top_idx.device).bool()[top_idx.clamp(min=0).long()] & (top_idx >= 0)
        ids_gpu = torch.where(on_cpu, torch.full_like(top_idx, -1), top_idx).to(torch.int32)
        ids_gpu_host = torch.where(on_cpu.cpu(), torch.full_like(ids_host, -1), ids_host).to(torch.int64)
        gpu_out = moe_offload_forward(flat, ids_gpu, top_w, cache, layer_id, ids_host=ids_gpu_host, **kw)
    except BaseException:
        job.discard()  # the worker must be done with x_h / out_h before they go, and its slot freed
        raise
    cpu_out = job.result()
    return (gpu_out.float() + cpu_out.to(flat.device, non_blocking=True)).to(flat.dtype)


__all__ = ["host_layer", "host_layer_from_bank", "cpu_moe_forward", "CpuJob", "split_experts", "moe_hybrid_forward"]
