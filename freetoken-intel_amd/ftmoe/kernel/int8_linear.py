"""Plain per-channel symmetric INT8 primitive (python/freetoken/kernel/triton/int8_linear.py):
unpacked int8 ``[N, K]`` weight + one scale per row.  Not a bank format of the
MoE path (the INT8 expert banks are the packed format of int8_packed_linear);
kept for API completeness as device-agnostic torch arithmetic."""
from __future__ import annotations

import torch

from ..quant import quantize_int8_channel  # noqa: F401  (int8_linear.py:34-43)


def dequantize_int8_channel(weight_int8: torch.Tensor, scale: torch.Tensor, *,
                            out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """int8_linear.py:46-60: ``fp32(q) * fp32(scale[row])`` rounded once."""
    if weight_int8.dtype != torch.int8:
        raise TypeError(f"weight_int8 must be int8, got {weight_int8.dtype}")
    if tuple(scale.shape) != tuple(weight_int8.shape[:-1]):
        raise ValueError(
            f"scale shape {tuple(scale.shape)} does not match weight_int8's row shape {tuple(weight_int8.shape[:-1])}"
        )
    return (weight_int8.to(torch.float32) * scale.unsqueeze(-1).to(torch.float32)).to(out_dtype)


def int8_linear(x: torch.Tensor, weight_int8: torch.Tensor, scale: torch.Tensor, *,
                bias: torch.Tensor | None = None) -> torch.Tensor:
    w = dequantize_int8_channel(weight_int8, scale, out_dtype=x.dtype)
    return torch.nn.functional.linear(x, w, bias)
