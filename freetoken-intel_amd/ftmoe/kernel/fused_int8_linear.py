"""Compressed-tensors pack-quantized INT8 projection against packed
``weight_packed``/``weight_scale`` (python/freetoken/kernel/triton/fused_int8_linear.py).

gfx950: offset-binary bytes are converted in registers to exact bf16 values
``byte - 128`` and each (row, group) scale is applied in fp32 to the group's
partial sum.  Groups that are neither a multiple of 64 nor the whole row (e.g.
32) run on the generic scalar HIP kernel."""
from __future__ import annotations

import torch

from ._common import run_expert, run_linear, single_proj


def _proj(weight_packed, weight_scale, k):
    n = weight_packed.shape[0]
    return single_proj("int8_channel", weight_packed, n, k, s=weight_scale, group=k // weight_scale.shape[1])


def fused_int8_linear(
    x: torch.Tensor,
    weight_packed: torch.Tensor,
    weight_scale: torch.Tensor,
    *,
    k: int,
    bias: torch.Tensor | None = None,
    block_m: int = 8,
    block_n: int = 16,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x @ dequantize_int8_packed(weight_packed, weight_scale, k=k).T (+ bias)``
    (fused_int8_linear.py:109-173 contract and checks)."""
    if weight_packed.dtype != torch.int32:
        raise TypeError(f"weight_packed must be int32, got {weight_packed.dtype}")
    m, kx = x.shape
    if kx != k:
        raise ValueError(f"x's K={kx} does not match the given k={k}")
    n, packed_cols = weight_packed.shape
    if weight_scale.shape[0] != n:
        raise ValueError(f"weight_packed/weight_scale row mismatch: {n} vs {weight_scale.shape[0]}")
    num_groups = weight_scale.shape[1]
    if k % num_groups != 0:
        raise ValueError(f"k={k} is not evenly divisible by num_groups={num_groups}")
    group_size = k // num_groups
    if group_size % 4 != 0:
        raise ValueError(f"group_size {group_size} (k={k} / num_groups={num_groups}) must be a multiple of 4")
    if group_size < 8:
        raise ValueError(f"group_size {group_size} is below the fused kernel's minimum of 8 (tl.dot's own hardware floor)")
    return run_linear(_proj(weight_packed, weight_scale, k), x, out_dtype=out_dtype, bias=bias)


def fused_int8_expert_forward(
    x: torch.Tensor,
    weight_packed_gate_up: torch.Tensor,
    weight_scale_gate_up: torch.Tensor,
    weight_packed_down: torch.Tensor,
    weight_scale_down: torch.Tensor,
    *,
    intermediate: int,
    k_gate_up: int,
    k_down: int,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """One expert's SwiGLU forward against packed INT8 banks (fused_int8_linear.py:176-201)."""
    return run_expert(_proj(weight_packed_gate_up, weight_scale_gate_up, k_gate_up),
                      _proj(weight_packed_down, weight_scale_down, k_down), x,
                      intermediate=intermediate, out_dtype=out_dtype)


# Reference crossover (fused_int8_linear.py:210), kept for API parity.
_FUSED_MAX_M = 64


def prefer_fused_over_dequant(m: int) -> bool:
    return m <= _FUSED_MAX_M
