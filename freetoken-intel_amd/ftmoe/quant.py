"""Weight quantizers and packers (generator side, load time -- not the hot path).

Torch restatements of the reference quantizers, runnable on any device, used to
build the packed banks the gfx950 kernels consume:

* :func:`quantize_block_fp8` -- python/freetoken/kernel/triton/fp8_block_linear.py:94-125
* :func:`quantize_mxfp4_blocks` -- python/freetoken/kernel/triton/mxfp4_linear.py:79-111
* :func:`quantize_int8_channel` -- python/freetoken/kernel/triton/int8_linear.py:34-43
* :func:`pack_int8_to_int32` -- inverse of unpack_int8_from_int32
  (python/freetoken/kernel/triton/int8_packed_linear.py:74-93): 4 offset-binary
  bytes (value + 128) per int32 along K, byte 0 = lowest k
* :func:`quantize_gptq_int4` -- the reference has no GPTQ quantizer; this is the
  AutoGPTQ-style symmetric round-to-nearest packer whose layout
  python/freetoken/kernel/triton/gptq_linear.py:18-30 dequantizes
  (scale = 2*amax/15 as fp16, q = clamp(round(w/scale) + 8, 0, 15), stored zero 7)
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn
_FP8_MAX = 448.0
_MXFP4_LUT = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)
_MXFP4_BLOCK = 32


def quantize_block_fp8(weight: torch.Tensor, *, block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """``[..., N, K]`` -> (float8_e4m3fn ``[..., N, K]``, fp32 scale ``[..., ceil(N/B), ceil(K/B)]``)."""
    if weight.ndim < 2:
        raise ValueError(f"weight must be at least 2-D [N, K], got shape {tuple(weight.shape)}")
    *lead, N, K = weight.shape
    nbr, nbc = -(-N // block), -(-K // block)
    w = weight.to(torch.float32)
    pad_n, pad_k = nbr * block - N, nbc * block - K
    if pad_n or pad_k:
        w = torch.nn.functional.pad(w, (0, pad_k, 0, pad_n))
    blocks = w.reshape(*lead, nbr, block, nbc, block)
    amax = blocks.abs().amax(dim=(-3, -1)).clamp_min(1e-12)
    scale = amax / _FP8_MAX
    q = (blocks / scale[..., :, None, :, None]).clamp(-_FP8_MAX, _FP8_MAX)
    q = q.reshape(*lead, nbr * block, nbc * block)[..., :N, :K].to(FP8)
    return q, scale


def quantize_mxfp4_blocks(weight: torch.Tensor, *, chunk_rows: int = 4096) -> tuple[torch.Tensor, torch.Tensor]:
    """``[..., K]`` (K a multiple of 32) -> (uint8 blocks ``[..., K/32, 16]``, uint8 e8m0 ``[..., K/32]``).

    Nearest-LUT-code search with ``argmin`` (first index on ties), processed in
    row chunks so the ``[rows, K/32, 32, 16]`` distance tensor stays small."""
    K = weight.shape[-1]
    if K % _MXFP4_BLOCK != 0:
        raise ValueError(f"MXFP4 quantization needs K a multiple of {_MXFP4_BLOCK}, got {K}")
    lead = weight.shape[:-1]
    rows = weight.reshape(-1, K)
    nb = K // _MXFP4_BLOCK
    lut = torch.tensor(_MXFP4_LUT, dtype=torch.float32, device=weight.device)
    blocks_out = torch.empty((rows.shape[0], nb, 16), dtype=torch.uint8, device=weight.device)
    scales_out = torch.empty((rows.shape[0], nb), dtype=torch.uint8, device=weight.device)
    for r0 in range(0, rows.shape[0], chunk_rows):
        w = rows[r0:r0 + chunk_rows].to(torch.float32)
        blocks_f = w.reshape(w.shape[0], nb, _MXFP4_BLOCK)
        amax = blocks_f.abs().amax(dim=-1).clamp_min(1e-12)
        exponent = torch.ceil(torch.log2(amax / 6.0))
        exponent_byte = exponent.add(127).round().clamp(0, 254).to(torch.uint8)
        scale = torch.exp2(exponent_byte.float() - 127).unsqueeze(-1)
        scaled = blocks_f / scale
        nibbles = (scaled.unsqueeze(-1) - lut).abs().argmin(dim=-1).to(torch.uint8)
        blocks_out[r0:r0 + chunk_rows] = nibbles[..., 0::2] | (nibbles[..., 1::2] << 4)
        scales_out[r0:r0 + chunk_rows] = exponent_byte
    return blocks_out.reshape(*lead, nb, 16), scales_out.reshape(*lead, nb)


def quantize_int8_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric INT8: (int8 ``weight.shape``, fp32 scale ``weight.shape[:-1]``)."""
    w = weight.to(torch.float32)
    amax = w.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
    scale = amax / 127
    q = (w / scale).round().clamp(-127, 127).to(torch.int8)
    return q, scale.squeeze(-1)


def pack_int8_to_int32(codes: torch.Tensor) -> torch.Tensor:
    """int8 ``[..., K]`` (K % 4 == 0) -> int32 ``[..., K/4]``, byte i of word c = code[4c+i] + 128."""
    K = codes.shape[-1]
    if K % 4 != 0:
        raise ValueError(f"K={K} must be a multiple of 4 to pack")
    b = (codes.to(torch.int64) + 128).reshape(*codes.shape[:-1], K // 4, 4)
    word = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)
    word = torch.where(word >= (1 << 31), word - (1 << 32), word)
    return word.to(torch.int32)


def _pack_nibbles_along(q: torch.Tensor, dim: int) -> torch.Tensor:
    """Pack 8 uint4 values per int32 along ``dim`` (LSB = first), as AutoGPTQ does."""
    q = q.movedim(dim, -1).to(torch.int64)
    *lead, n = q.shape
    q = q.reshape(*lead, n // 8, 8)
    shifts = torch.arange(0, 32, 4, dtype=torch.int64, device=q.device)
    word = (q << shifts).sum(dim=-1)
    word = torch.where(word >= (1 << 31), word - (1 << 32), word).to(torch.int32)
    return word.movedim(-1, dim)


def quantize_gptq_int4(weight_kn: torch.Tensor, *, group_size: int = 128
                       ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Symmetric int4, ``desc_act=False``: ``[..., K, N]`` (in, out) ->
    (qweight int32 ``[..., K/8, N]``, qzeros int32 ``[..., K/g, N/8]``, scales fp16 ``[..., K/g, N]``)."""
    *lead, K, N = weight_kn.shape
    if K % group_size != 0 or group_size % 8 != 0 or N % 8 != 0:
        raise ValueError(f"need K % group_size == 0, group_size % 8 == 0, N % 8 == 0 (K={K}, N={N}, g={group_size})")
    G = K // group_size
    w = weight_kn.to(torch.float32).reshape(*lead, G, group_size, N)
    amax = w.abs().amax(dim=-2).clamp_min(1e-12)  # [..., G, N]
    scales = (2.0 * amax / 15.0).to(torch.float16)
    q = torch.clamp(torch.round(w / scales.to(torch.float32).unsqueeze(-2)) + 8, 0, 15)
    q = q.reshape(*lead, K, N).to(torch.int32)
    qweight = _pack_nibbles_along(q, dim=-2)  # [..., K/8, N]
    zeros = torch.full((*lead, G, N), 7, dtype=torch.int32, device=weight_kn.device)
    qzeros = _pack_nibbles_along(zeros, dim=-1)  # [..., G, N/8]
    return qweight, qzeros, scales
