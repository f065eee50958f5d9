"""Shared launch helpers for the per-projection drop-in API."""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _native as nat
from ..banks import Proj, single_proj
from ..layer import MoeLayer


def run_linear(proj: Proj, x: torch.Tensor, *, out_dtype: Optional[torch.dtype],
               bias: Optional[torch.Tensor]) -> torch.Tensor:
    """``cast(x @ deq(W).T, out_dtype) (+ bias)`` on the GPU via ``ftm_linear``.

    fp32 accumulation; the bias is added after the cast with torch's type
    promotion, as python/freetoken/kernel/triton/fused_fp8_linear.py:148-151 does."""
    nat.require_gpu(x, "x")
    for t in proj.tensors():
        nat.require_gpu(t, "weight")
    if bias is not None:
        nat.require_gpu(bias, "bias")
    x = x.contiguous()
    M = x.shape[0]
    out_dtype = out_dtype if out_dtype is not None else x.dtype
    final = torch.promote_types(out_dtype, bias.dtype) if bias is not None else out_dtype
    out = torch.empty((M, proj.N), dtype=final, device=x.device)
    if M == 0:
        return out
    b = bias.contiguous() if bias is not None else None
    rc = nat.lib().ftm_linear(ctypes.byref(proj.c()), 0, x.data_ptr(), nat.dtype_code(x.dtype), M, out.data_ptr(),
                              nat.dtype_code(out_dtype), nat.ptr(b), nat.dtype_code(b.dtype) if b is not None else 0,
                              nat.dtype_code(final), nat.stream_of(x))
    nat.check(rc, "ftm_linear")
    return out


def run_expert(gate_up: Proj, down: Proj, x: torch.Tensor, *, intermediate: int,
               out_dtype: Optional[torch.dtype]) -> torch.Tensor:
    """``down(silu(gate(x)) * up(x))`` for one packed expert, w13 + activation +
    w2 fused in the HIP layer kernels: ``gu`` in fp32, ``h`` rounded to
    ``out_dtype`` (default ``x.dtype``), fp32 down projection rounded to
    ``out_dtype`` -- the reference's two fused calls
    (python/freetoken/kernel/triton/fused_fp8_linear.py:172-175).  bf16 in and
    out runs the bf16 layer kernels; any other pair runs them on fp32
    activations (``x`` widened exactly) with ``h`` rounded to ``out_dtype``."""
    nat.require_gpu(x, "x")
    out_dtype = out_dtype if out_dtype is not None else x.dtype
    if x.dtype == torch.bfloat16 and out_dtype == torch.bfloat16:
        act_dtype, h_dtype = torch.bfloat16, None
    else:
        act_dtype, h_dtype = torch.float32, out_dtype
    xa = x.to(act_dtype).contiguous()
    layer = MoeLayer(w13=gate_up, w2=down, num_experts=1, hidden=gate_up.K, inter=intermediate, topk=1,
                     act="silu", act_dtype=act_dtype, h_dtype=h_dtype)
    y = layer.expert_forward(0, xa)
    return y if y.dtype == out_dtype else y.to(out_dtype)


__all__ = ["run_linear", "run_expert", "single_proj"]
