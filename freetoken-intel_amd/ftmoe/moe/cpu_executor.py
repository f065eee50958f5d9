"""Host-side routed-expert executor: the drop-in for the reference's
``CpuMoeExecutor`` (python/freetoken/moe/cpu_executor.py:51-144).

Same constructor (``num_experts, intermediate, *, threads=0``) and the same
``forward(flat, top_idx, top_w, gate_up, down) -> [T, H]`` contract: the routed
contribution ``sum_j top_w[:, j] * expert_{top_idx[:, j]}(flat)`` computed on
the host from the layer's host banks (``gate_up [E, 2I, H]``, gate rows first;
``down [E, H, I]``), returned on ``flat``'s device in ``flat``'s dtype.

The GEMM is this library's CPU kernel (``ftm_cpu_moe_forward``, csrc/ftm_cpu.cpp:
AVX-512 where the host has it, experts in contiguous ranges over ``threads``
host threads, fp32 gate/up, fp32 ``h``, fp32 down projection, each thread's
partial sums added in thread order) -- the arithmetic of the reference's
native ``cpu_moe_forward_fast``.  ``threads=0`` uses every host thread,
clamped to the expert count, as the reference's pool does.  There is no
pure-Python fallback: the library is part of this package, so a missing
library raises instead.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _native as nat
from ..banks import Proj
from .hybrid import cpu_moe_forward


def _dense_layer(gate_up: torch.Tensor, down: torch.Tensor, num_experts: int, intermediate: int, topk: int):
    """``ftm_moe_layer`` over dense host banks (bf16 as stored, any other float
    dtype as fp32) and what must stay alive while it is used."""
    if gate_up.dim() != 3 or down.dim() != 3:
        raise ValueError(f"gate_up must be [E, 2I, H] and down [E, H, I], got {tuple(gate_up.shape)} and "
                         f"{tuple(down.shape)}")
    E, I2, H = gate_up.shape
    if E != num_experts or I2 != 2 * intermediate or tuple(down.shape) != (E, H, intermediate):
        raise ValueError(f"banks gate_up {tuple(gate_up.shape)} / down {tuple(down.shape)} do not match "
                         f"num_experts={num_experts}, intermediate={intermediate}")
    if gate_up.dtype == torch.bfloat16 and down.dtype == torch.bfloat16:
        fmt, gu, dn = "bf16", gate_up.to("cpu").contiguous(), down.to("cpu").contiguous()
    else:
        fmt, gu, dn = "fp32", gate_up.to("cpu", torch.float32).contiguous(), down.to("cpu", torch.float32).contiguous()
    w13, w2 = Proj(fmt, gu, 2 * intermediate, H), Proj(fmt, dn, H, intermediate)
    L = nat.FtmMoeLayer()
    L.w13, L.w2 = w13.c(), w2.c()
    L.num_experts, L.hidden, L.inter, L.topk = int(E), int(H), int(intermediate), int(topk)
    L.act = nat.ACT_SILU  # SiLU-gated: the reference executor's SwiGLU
    L.swiglu_alpha, L.swiglu_limit = 1.702, 7.0
    L.act_dtype = nat.DT_F32
    L.h_dtype = nat.DT_F32
    return L, (w13, w2, gu, dn)


class CpuMoeExecutor:
    """Routed experts on the host over the layer's host banks (see the module
    docstring).  Owns no model state; one instance serves every layer."""

    def __init__(self, num_experts: int, intermediate: int, *, threads: int = 0) -> None:
        self.num_experts = int(num_experts)
        self.intermediate = int(intermediate)
        self.threads = int(threads)
        # the layer descriptor of the banks seen last (rebuilt when they change)
        self._cached: Optional[tuple] = None

    def _layer(self, gate_up: torch.Tensor, down: torch.Tensor, topk: int):
        key = (gate_up.data_ptr(), down.data_ptr(), gate_up.dtype, down.dtype, tuple(gate_up.shape), int(topk),
               gate_up.device.type, down.device.type)
        if self._cached is None or self._cached[0] != key or gate_up.device.type != "cpu":
            self._cached = (key, *_dense_layer(gate_up, down, self.num_experts, self.intermediate, topk))
        return self._cached[1]

    def forward(self, flat: torch.Tensor, top_idx: torch.Tensor, top_w: torch.Tensor, gate_up: torch.Tensor,
                down: torch.Tensor) -> torch.Tensor:
        """``flat [T, H]``, ``top_idx [T, k]`` expert ids, ``top_w [T, k]`` router
        weights, host banks ``gate_up [E, 2I, H]`` / ``down [E, H, I]`` ->
        ``[T, H]`` routed contribution on ``flat``'s device and dtype."""
        if flat.dim() != 2 or top_idx.dim() != 2 or top_idx.shape != top_w.shape or top_idx.shape[0] != flat.shape[0]:
            raise ValueError(f"flat {tuple(flat.shape)}, top_idx {tuple(top_idx.shape)} and top_w "
                             f"{tuple(top_w.shape)} do not describe one [T, H] batch with [T, k] routing")
        if flat.shape[0] == 0:
            return torch.zeros_like(flat)
        layer = self._layer(gate_up, down, top_idx.shape[1])
        out = cpu_moe_forward(layer, flat, top_idx, top_w, threads=self.threads)
        return out.to(device=flat.device, dtype=flat.dtype)

    __call__ = forward


__all__ = ["CpuMoeExecutor"]
