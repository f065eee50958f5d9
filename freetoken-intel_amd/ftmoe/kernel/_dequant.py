"""Dense dequantization of one packed matrix through ``ftm_dequant`` (HIP)."""
from __future__ import annotations

import ctypes

import torch

from .. import _native as nat
from ..banks import Proj


def dequant(proj: Proj, *, out_dtype: torch.dtype, transpose: bool = False, slot: int = 0) -> torch.Tensor:
    """``[N, K]`` (or ``[K, N]`` with ``transpose``) of ``out_dtype``: the reference's
    fp32 product rounded once (bit-exact)."""
    for t in proj.tensors():
        nat.require_gpu(t, "weight")
    shape = (proj.K, proj.N) if transpose else (proj.N, proj.K)
    out = torch.empty(shape, dtype=out_dtype, device=proj.device)
    rc = nat.lib().ftm_dequant(ctypes.byref(proj.c()), int(slot), out.data_ptr(), nat.dtype_code(out_dtype),
                               1 if transpose else 0, torch.cuda.current_stream(proj.device).cuda_stream)
    nat.check(rc, "ftm_dequant")
    return out
