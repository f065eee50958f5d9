"""GPTQ int4 weights: dequantize / dequant-then-matmul
(python/freetoken/kernel/triton/gptq_linear.py).

``weight[k, n] = scales[g_idx[k], n] * (q[k, n] - (qzeros[g_idx[k], n] + 1))``
computed on the GPU by ``ftm_dequant``.  Like the reference's fused path, only
sequential groups (``desc_act=False``: ``g_idx[k] = k // group_size``) are
supported; any other ``g_idx`` raises."""
from __future__ import annotations

import torch

from ..banks import single_proj
from ._dequant import dequant

_BITS = 4


def _check(qweight, qzeros, scales):
    if qweight.dtype != torch.int32:
        raise TypeError(f"qweight must be int32, got {qweight.dtype}")
    if qzeros.dtype != torch.int32:
        raise TypeError(f"qzeros must be int32, got {qzeros.dtype}")
    k_packed, n = qweight.shape
    if scales.shape[1] != n or qzeros.shape[1] * (32 // _BITS) != n:
        raise ValueError(
            f"qweight/qzeros/scales shape mismatch: qweight={tuple(qweight.shape)}, "
            f"qzeros={tuple(qzeros.shape)}, scales={tuple(scales.shape)}"
        )
    return k_packed * (32 // _BITS), n


def dequantize_gptq_int4_sequential_groups(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, *,
                                           group_size: int, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dense ``[K, N]`` (in, out) for ``desc_act=False`` (gptq_linear.py:102-124)."""
    k, n = _check(qweight, qzeros, scales)
    proj = single_proj("gptq_int4", qweight, n, k, s=scales, z=qzeros, group=group_size)
    return dequant(proj, out_dtype=out_dtype, transpose=True)


def dequantize_gptq_int4(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, g_idx: torch.Tensor, *,
                         out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dense ``[K, N]`` (gptq_linear.py:55-99); ``g_idx`` must be sequential groups."""
    if g_idx.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"g_idx must be an integer tensor, got {g_idx.dtype}")
    k, n = _check(qweight, qzeros, scales)
    if g_idx.shape[0] != k:
        raise ValueError(f"g_idx length {g_idx.shape[0]} does not match qweight's implied K={k}")
    groups = qzeros.shape[0]
    group_size = -(-k // groups)
    expected = torch.arange(k, device=g_idx.device, dtype=torch.int64) // group_size
    if not torch.equal(g_idx.to(torch.int64), expected):
        raise NotImplementedError("only sequential GPTQ groups (desc_act=False) are supported on gfx950")
    return dequantize_gptq_int4_sequential_groups(qweight, qzeros, scales, group_size=group_size, out_dtype=out_dtype)


def gptq_linear(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                g_idx: torch.Tensor, *, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ dequantize_gptq_int4(...).T (+ bias)`` (gptq_linear.py:127-143)."""
    w = dequantize_gptq_int4(qweight, qzeros, scales, g_idx, out_dtype=x.dtype)
    return torch.nn.functional.linear(x, w.T, bias)
