"""Block-FP8 projection against packed ``weight_fp8``/``weight_scale_inv``, never
materialising the dense weight (python/freetoken/kernel/triton/fused_fp8_linear.py).

gfx950: e4m3 bytes are converted in registers to their exact bf16 values
(``v_cvt_scalef32_pk_bf16_fp8``, scale 1.0), multiplied on the bf16 matrix
core, and each 128x128 block's fp32 scale is applied to the block's partial
sum.  Activations in fp32/fp16 are split into bf16 hi + lo halves so the
product keeps ~16 significant bits (the reference's tl.dot runs in fp32).
e5m2 weights (accepted by the reference, fused_fp8_linear.py:123) run on the
generic GPU kernels with the same fp32 arithmetic."""
from __future__ import annotations

import torch

from ._common import run_expert, run_linear, single_proj

_QBLOCK = 128


def _proj(weight_fp8: torch.Tensor, weight_scale_inv: torch.Tensor, block: int):
    n, k = weight_fp8.shape
    fmt = "fp8_e5m2_block" if weight_fp8.dtype == torch.float8_e5m2 else "fp8_block"
    return single_proj(fmt, weight_fp8, n, k, s=weight_scale_inv, group=block)


def fused_fp8_linear(
    x: torch.Tensor,
    weight_fp8: torch.Tensor,
    weight_scale_inv: torch.Tensor,
    *,
    bias: torch.Tensor | None = None,
    block: int = _QBLOCK,
    block_m: int = 1,
    block_n: int = 16,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x @ dequantize_block_fp8(weight_fp8, weight_scale_inv).T (+ bias)``.

    Same contract and checks as the reference (fused_fp8_linear.py:95-151);
    ``block_m`` / ``block_n`` are the reference's Triton tile knobs, validated
    but not used (the gfx950 tiling is fixed)."""
    if block % block_n != 0:
        raise ValueError(f"block_n {block_n} must divide block {block} evenly")
    if weight_fp8.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise TypeError(f"weight_fp8 must be an fp8 dtype, got {weight_fp8.dtype}")
    m, k = x.shape
    n, k2 = weight_fp8.shape
    if k != k2:
        raise ValueError(f"x's K={k} does not match weight_fp8's K={k2}")
    expected_scale_shape = (-(-n // block), -(-k // block))
    if tuple(weight_scale_inv.shape) != expected_scale_shape:
        raise ValueError(
            f"weight_scale_inv shape {tuple(weight_scale_inv.shape)} does not match "
            f"the expected {expected_scale_shape} for weight_fp8 shape {(n, k)} at block={block}"
        )
    return run_linear(_proj(weight_fp8, weight_scale_inv, block), x, out_dtype=out_dtype, bias=bias)


def fused_fp8_expert_forward(
    x: torch.Tensor,
    weight_fp8_gate_up: torch.Tensor,
    weight_scale_inv_gate_up: torch.Tensor,
    weight_fp8_down: torch.Tensor,
    weight_scale_inv_down: torch.Tensor,
    *,
    intermediate: int,
    block: int = _QBLOCK,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """One expert's SwiGLU forward against packed block-FP8 banks
    (fused_fp8_linear.py:154-175): gu in fp32, h = silu(gate) * up rounded to
    ``out_dtype`` (default ``x.dtype``), then the down projection."""
    return run_expert(_proj(weight_fp8_gate_up, weight_scale_inv_gate_up, block),
                      _proj(weight_fp8_down, weight_scale_inv_down, block), x,
                      intermediate=intermediate, out_dtype=out_dtype)


# Rows-per-expert crossover kept from the reference (fused_fp8_linear.py:183)
# for API parity; the gfx950 engine itself serves any row count.
_FUSED_MAX_M = 8


def prefer_fused_over_dequant(m: int) -> bool:
    """Whether the fused path is preferred for ``m`` rows (reference rule, M <= 8)."""
    return m <= _FUSED_MAX_M
