"""MXFP4 projection against packed ``blocks``/``scales``
(python/freetoken/kernel/triton/fused_mxfp4_linear.py).

gfx950: one 16-byte load per lane is exactly one 32-element block of one row;
``v_cvt_scalef32_pk_bf16_fp4`` decodes two e2m1 nibbles per instruction and
applies the block's e8m0 factor, exactly (LUT * 2^e fits bf16)."""
from __future__ import annotations

import torch

from ._common import run_expert, run_linear, single_proj

_QBLOCK = 32


def _proj(blocks, scales):
    n, nb, _ = blocks.shape
    return single_proj("mxfp4", blocks, n, nb * _QBLOCK, s=scales, group=_QBLOCK)


def fused_mxfp4_linear(
    x: torch.Tensor,
    weight_blocks: torch.Tensor,
    weight_scales: torch.Tensor,
    *,
    bias: torch.Tensor | None = None,
    block_m: int = 8,
    block_n: int = 16,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x @ dequantize_mxfp4_blocks(weight_blocks, weight_scales).T (+ bias)``
    (fused_mxfp4_linear.py:129-188 contract and checks)."""
    if weight_blocks.dtype != torch.uint8:
        raise TypeError(f"weight_blocks must be uint8, got {weight_blocks.dtype}")
    if weight_scales.dtype != torch.uint8:
        raise TypeError(f"weight_scales must be uint8, got {weight_scales.dtype}")
    if weight_blocks.shape[-1] != 16:
        raise ValueError(f"weight_blocks' last dim must be 16 packed bytes, got {weight_blocks.shape[-1]}")
    m, k = x.shape
    n, n_blocks, _ = weight_blocks.shape
    if n_blocks * _QBLOCK != k:
        raise ValueError(f"x's K={k} does not match weight_blocks' implied K={n_blocks * _QBLOCK}")
    if tuple(weight_scales.shape) != (n, n_blocks):
        raise ValueError(
            f"weight_scales shape {tuple(weight_scales.shape)} does not match weight_blocks' implied {(n, n_blocks)}"
        )
    return run_linear(_proj(weight_blocks, weight_scales), x, out_dtype=out_dtype, bias=bias)


def fused_mxfp4_expert_forward(
    x: torch.Tensor,
    blocks_gate_up: torch.Tensor,
    scales_gate_up: torch.Tensor,
    blocks_down: torch.Tensor,
    scales_down: torch.Tensor,
    *,
    intermediate: int,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """One expert's SwiGLU forward against packed MXFP4 banks (fused_mxfp4_linear.py:191-210)."""
    return run_expert(_proj(blocks_gate_up, scales_gate_up), _proj(blocks_down, scales_down), x,
                      intermediate=intermediate, out_dtype=out_dtype)


# Reference bound (fused_mxfp4_linear.py:218), kept for API parity.
_FUSED_MAX_M = 128


def prefer_fused_over_dequant(m: int) -> bool:
    return m <= _FUSED_MAX_M
