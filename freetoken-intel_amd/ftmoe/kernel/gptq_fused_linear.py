"""GPTQ int4 (g128, desc_act=False) projection against packed
``qweight``/``qzeros``/``scales`` (python/freetoken/kernel/triton/gptq_fused_linear.py).

gfx950: each int32 word of 8 nibbles becomes 8 bf16 values ``128 + q`` with
two bit operations per pair (the nibble sits in the mantissa of bf16 128.0),
the matrix core accumulates x . (128 + q) per group, and the group's zero
point and the 128 bias are removed in fp32 as ``s * (acc - (128 + z + 1) * sum(x))``."""
from __future__ import annotations

import torch

from ._common import run_expert, run_linear, single_proj

_BITS = 4
_P = 32 // _BITS


def _proj(qweight, qzeros, scales, group_size):
    k_packed, n = qweight.shape
    return single_proj("gptq_int4", qweight, n, k_packed * _P, s=scales, z=qzeros, group=group_size)


def fused_gptq_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    qzeros: torch.Tensor,
    scales: torch.Tensor,
    *,
    group_size: int,
    bias: torch.Tensor | None = None,
    block_m: int = 8,
    block_n: int = 16,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x @ dequantize_gptq_int4_sequential_groups(...).T (+ bias)``
    (gptq_fused_linear.py:131-196 contract and checks)."""
    if group_size % _P != 0:
        raise ValueError(f"group_size {group_size} must be a multiple of {_P} (the int4 packing factor)")
    if qweight.dtype != torch.int32:
        raise TypeError(f"qweight must be int32, got {qweight.dtype}")
    if qzeros.dtype != torch.int32:
        raise TypeError(f"qzeros must be int32, got {qzeros.dtype}")
    m, k = x.shape
    k_packed, n = qweight.shape
    if k_packed * _P != k:
        raise ValueError(f"x's K={k} does not match qweight's implied K={k_packed * _P}")
    if scales.shape[1] != n or qzeros.shape[1] * _P != n:
        raise ValueError(
            f"qweight/qzeros/scales shape mismatch: qweight={tuple(qweight.shape)}, "
            f"qzeros={tuple(qzeros.shape)}, scales={tuple(scales.shape)}"
        )
    return run_linear(_proj(qweight, qzeros, scales, group_size), x, out_dtype=out_dtype, bias=bias)


def fused_gptq_expert_forward(
    x: torch.Tensor,
    qweight_gate_up: torch.Tensor,
    qzeros_gate_up: torch.Tensor,
    scales_gate_up: torch.Tensor,
    qweight_down: torch.Tensor,
    qzeros_down: torch.Tensor,
    scales_down: torch.Tensor,
    *,
    group_size: int,
    intermediate: int,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """One expert's SwiGLU forward against packed GPTQ banks (gptq_fused_linear.py:199-230)."""
    return run_expert(_proj(qweight_gate_up, qzeros_gate_up, scales_gate_up, group_size),
                      _proj(qweight_down, qzeros_down, scales_down, group_size), x,
                      intermediate=intermediate, out_dtype=out_dtype)


# Reference crossover (gptq_fused_linear.py:240), kept for API parity.
_FUSED_MAX_M = 32


def prefer_fused_over_dequant(m: int) -> bool:
    return m <= _FUSED_MAX_M
