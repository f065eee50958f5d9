"""Compressed-tensors pack-quantized INT8 weights
(python/freetoken/kernel/triton/int8_packed_linear.py): 4 offset-binary bytes
per int32 along K (stored byte = value + 128), per-(row, group) scales."""
from __future__ import annotations

import torch

from ..banks import single_proj
from ..quant import pack_int8_to_int32  # noqa: F401  (the inverse packer)
from ._dequant import dequant

_BITS = 8
_ELEMS_PER_WORD = 32 // _BITS
_OFFSET = 1 << (_BITS - 1)


def unpack_int8_from_int32(weight_packed: torch.Tensor, k: int) -> torch.Tensor:
    """``[N, ceil(K/4)]`` int32 -> ``[N, K]`` int8 (int8_packed_linear.py:74-93)."""
    if weight_packed.dtype != torch.int32:
        raise TypeError(f"weight_packed must be int32, got {weight_packed.dtype}")
    n, packed_cols = weight_packed.shape
    shifts = torch.arange(0, 32, 8, device=weight_packed.device, dtype=torch.int32)
    b = (weight_packed.unsqueeze(-1) >> shifts) & 0xFF
    return (b.reshape(n, packed_cols * _ELEMS_PER_WORD)[:, :k] - _OFFSET).to(torch.int8)


def dequantize_int8_packed(weight_packed: torch.Tensor, weight_scale: torch.Tensor, *, k: int,
                           out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dense ``[N, K]`` (int8_packed_linear.py:96-125), on the GPU."""
    n, packed_cols = weight_packed.shape
    if weight_scale.shape[0] != n:
        raise ValueError(f"weight_packed/weight_scale row mismatch: {n} vs {weight_scale.shape[0]}")
    num_groups = weight_scale.shape[1]
    if k % num_groups != 0:
        raise ValueError(f"K={k} is not evenly divisible by num_groups={num_groups}")
    if weight_packed.dtype != torch.int32:
        raise TypeError(f"weight_packed must be int32, got {weight_packed.dtype}")
    proj = single_proj("int8_channel", weight_packed, n, k, s=weight_scale, group=k // num_groups)
    return dequant(proj, out_dtype=out_dtype)
