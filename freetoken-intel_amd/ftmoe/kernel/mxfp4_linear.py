"""OCP MXFP4 weights (python/freetoken/kernel/triton/mxfp4_linear.py): 32 e2m1
values per block, 16 bytes, low nibble = even element, one e8m0 byte per block:
``value = LUT[nibble] * 2 ** (e8m0 - 127)`` computed on the GPU by ``ftm_dequant``."""
from __future__ import annotations

import torch

from ..banks import single_proj
from ..quant import quantize_mxfp4_blocks  # noqa: F401  (mxfp4_linear.py:79-111)
from ._dequant import dequant


def dequantize_mxfp4_blocks(blocks: torch.Tensor, scales: torch.Tensor, *,
                            out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dense ``[..., K]`` from ``blocks [..., n_blocks, 16]`` + ``scales [..., n_blocks]`` (mxfp4_linear.py:46-76)."""
    if blocks.dtype != torch.uint8:
        raise TypeError(f"MXFP4 blocks must be uint8, got {blocks.dtype}")
    if scales.dtype != torch.uint8:
        raise TypeError(f"MXFP4 scales must be uint8, got {scales.dtype}")
    if blocks.shape[-1] != 16:
        raise ValueError(f"MXFP4 block pack dimension must be 16 bytes, got {blocks.shape[-1]}")
    if blocks.shape[:-1] != scales.shape:
        raise ValueError(f"MXFP4 blocks/scales shape mismatch: {tuple(blocks.shape[:-1])} vs {tuple(scales.shape)}")
    lead = blocks.shape[:-2]
    nb = blocks.shape[-2]
    rows = 1
    for d in lead:
        rows *= d
    b2 = blocks.reshape(rows, nb, 16).contiguous()
    s2 = scales.reshape(rows, nb).contiguous()
    out = dequant(single_proj("mxfp4", b2, rows, nb * 32, s=s2, group=32), out_dtype=out_dtype)
    return out.reshape(*lead, nb * 32)


def mxfp4_linear(x: torch.Tensor, weight_blocks: torch.Tensor, weight_scales: torch.Tensor, *,
                 bias: torch.Tensor | None = None) -> torch.Tensor:
    w = dequantize_mxfp4_blocks(weight_blocks, weight_scales, out_dtype=x.dtype)
    return torch.nn.functional.linear(x, w, bias)
