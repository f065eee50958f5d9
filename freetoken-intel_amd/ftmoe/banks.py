"""Projection-bank descriptors: torch tensors -> ``ftm_proj`` (include/ftmoe.h).

Bank layouts are the reference's packed per-expert row layouts
(python/freetoken/moe/offload_cache.py:140-173), one leading slot axis:

================  =====================================================  ===========================
format            weight (per slot)                                      scales / zeros (per slot)
================  =====================================================  ===========================
``bf16``          bf16 ``[N, K]``                                        --
``fp8_block``     float8_e4m3fn ``[N, K]``                               ``[ceil(N/B), ceil(K/B)]``
``gptq_int4``     int32 qweight ``[K/8, N]``                             qzeros ``[K/g, N/8]`` int32, scales ``[K/g, N]``
``int8_channel``  int32 ``[N, K/4]`` (offset-binary bytes)                ``[N, K/group]``
``mxfp4``         uint8 blocks ``[N, K/32, 16]``                         uint8 e8m0 ``[N, K/32]``
================  =====================================================  ===========================
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _native as nat

FORMATS = {
    "bf16": nat.FMT_BF16,
    "fp8_block": nat.FMT_FP8_BLOCK,
    "gptq_int4": nat.FMT_GPTQ_INT4,
    "int8_channel": nat.FMT_INT8_PACKED,
    "mxfp4": nat.FMT_MXFP4,
    "fp32": nat.FMT_FP32,
    "fp8_e5m2_block": nat.FMT_FP8_E5M2_BLOCK,
}


def _slot_stride_bytes(t: Optional[torch.Tensor], slotted: bool) -> int:
    if t is None or not slotted:
        return 0
    return t.stride(0) * t.element_size()


def _scale_dtype(t: Optional[torch.Tensor]) -> int:
    if t is None or t.dtype == torch.uint8:
        return nat.DT_F32
    return nat.dtype_code(t.dtype)


@dataclass
class Proj:
    """One projection bank, ``[num_slots, N, K]`` logical (or a single matrix)."""

    fmt: str
    w: torch.Tensor
    N: int
    K: int
    s: Optional[torch.Tensor] = None
    z: Optional[torch.Tensor] = None
    bias: Optional[torch.Tensor] = None
    group: int = 0
    slotted: bool = True
    flags: int = 0  # ftm_proj.flags (nat.PROJ_RING_B)
    _c: Optional[nat.FtmProj] = field(default=None, repr=False)

    def __post_init__(self) -> None:
        if self.fmt not in FORMATS:
            raise ValueError(f"unknown bank format {self.fmt!r}")
        for name in ("w", "s", "z", "bias"):
            t = getattr(self, name)
            if t is not None and not t.is_contiguous():
                setattr(self, name, t.contiguous())

    @property
    def num_slots(self) -> int:
        return self.w.shape[0] if self.slotted else 1

    @property
    def device(self) -> torch.device:
        return self.w.device

    def c(self) -> nat.FtmProj:
        if self._c is None:
            p = nat.FtmProj()
            p.w = self.w.data_ptr()
            p.s = self.s.data_ptr() if self.s is not None else None
            p.z = self.z.data_ptr() if self.z is not None else None
            p.bias = self.bias.data_ptr() if self.bias is not None else None
            p.w_stride = _slot_stride_bytes(self.w, self.slotted)
            p.s_stride = _slot_stride_bytes(self.s, self.slotted)
            p.z_stride = _slot_stride_bytes(self.z, self.slotted)
            p.bias_stride = _slot_stride_bytes(self.bias, self.slotted)
            p.fmt = FORMATS[self.fmt]
            p.s_dtype = _scale_dtype(self.s)
            p.bias_dtype = nat.dtype_code(self.bias.dtype) if self.bias is not None else nat.DT_BF16
            p.group = int(self.group)
            p.N = int(self.N)
            p.K = int(self.K)
            p.num_slots = int(self.num_slots)
            p.flags = int(self.flags)
            self._c = p
        return self._c

    def tensors(self):
        return [t for t in (self.w, self.s, self.z, self.bias) if t is not None]


def proj_from_bank(fmt: str, bank: dict, *, which: str, N: int, K: int, group: Optional[int] = None,
                   bias: Optional[torch.Tensor] = None, slotted: bool = True) -> Proj:
    """Build a :class:`Proj` from a reference bank dict (``_BANK_SCHEMAS`` names)
    for ``which`` in ``("gate_up", "down")``."""
    if fmt == "bf16":
        return Proj(fmt, bank[which], N, K, bias=bias, slotted=slotted)
    if fmt == "fp8_block":
        return Proj(fmt, bank[f"weight_{which}"], N, K, s=bank[f"scale_{which}"], bias=bias,
                    group=group or 128, slotted=slotted)
    if fmt == "gptq_int4":
        if group is None:
            raise ValueError("gptq_int4 needs group_size (refuse to guess, offload_cache.py:748-764)")
        return Proj(fmt, bank[f"qweight_{which}"], N, K, s=bank[f"scales_{which}"], z=bank[f"qzeros_{which}"],
                    bias=bias, group=group, slotted=slotted)
    if fmt == "int8_channel":
        s = bank[f"weight_scale_{which}"]
        num_groups = s.shape[-1]
        if K % num_groups != 0:
            raise ValueError(f"K={K} is not evenly divisible by num_groups={num_groups}")
        return Proj(fmt, bank[f"weight_packed_{which}"], N, K, s=s, bias=bias, group=K // num_groups,
                    slotted=slotted)
    if fmt == "mxfp4":
        return Proj(fmt, bank[f"blocks_{which}"], N, K, s=bank[f"scales_{which}"], bias=bias, group=32,
                    slotted=slotted)
    raise ValueError(f"unknown bank format {fmt!r}")


def single_proj(fmt: str, w: torch.Tensor, N: int, K: int, *, s=None, z=None, group: int = 0) -> Proj:
    """One matrix (no slot axis), for the per-projection ``fused_*_linear`` API."""
    return Proj(fmt, w, N, K, s=s, z=z, group=group, slotted=False)
