"""Block-FP8 weights: dequantize / quantize / dequant-then-matmul
(python/freetoken/kernel/triton/fp8_block_linear.py).

``weight_bf16[i, j] = weight_fp8[i, j] * weight_scale_inv[i // block, j // block]``
computed on the GPU by ``ftm_dequant`` (fp32 product, one rounding)."""
from __future__ import annotations

import torch

from ..banks import single_proj
from ..quant import FP8, quantize_block_fp8  # noqa: F401  (re-exported, fp8_block_linear.py:94-125)
from ._dequant import dequant

_BLOCK = 128


def dequantize_block_fp8(weight_fp8: torch.Tensor, weight_scale_inv: torch.Tensor, *, block: int = _BLOCK,
                         out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dense ``[N, K]`` from block-quantized fp8 + scales (fp8_block_linear.py:48-91)."""
    if weight_fp8.ndim != 2:
        raise ValueError(f"weight_fp8 must be 2-D [N, K], got shape {tuple(weight_fp8.shape)}")
    N, K = weight_fp8.shape
    expected = ((N + block - 1) // block, (K + block - 1) // block)
    if tuple(weight_scale_inv.shape) != expected:
        raise ValueError(
            f"weight_scale_inv shape {tuple(weight_scale_inv.shape)} does not match "
            f"the expected {expected} for weight_fp8 shape {(N, K)} at block={block}"
        )
    if weight_fp8.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise TypeError(f"weight_fp8 must be float8_e4m3fn or float8_e5m2, got {weight_fp8.dtype}")
    fmt = "fp8_e5m2_block" if weight_fp8.dtype == torch.float8_e5m2 else "fp8_block"
    return dequant(single_proj(fmt, weight_fp8, N, K, s=weight_scale_inv, group=block), out_dtype=out_dtype)


def fp8_block_linear(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale_inv: torch.Tensor, *,
                     block: int = _BLOCK, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ dequantize_block_fp8(...).T (+ bias)``: GPU dequant, then the library GEMM."""
    w = dequantize_block_fp8(weight_fp8, weight_scale_inv, block=block, out_dtype=x.dtype)
    return torch.nn.functional.linear(x, w, bias)
