"""GPU: dequantization and the in-register decode paths are bit-exact.

* ``ftm_dequant`` against the oracle for every format, every code value
  (all 256 e4m3 bytes, all 256 MXFP4 bytes incl. the e8m0 edge exponents),
  and bf16 / fp16 / fp32 outputs;
* the MFMA engines' register decode (``v_cvt_scalef32_pk_bf16_fp8/fp4``, the
  GPTQ 0x4300 nibble trick, the INT8 offset) through ``ftm_linear`` with an
  identity activation: ``eye(K) @ W^T`` must reproduce the dequantized weight
  exactly, because every product is one exact fp32 multiply.
"""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import np_

from ftmoe.banks import single_proj
from ftmoe.kernel._common import run_linear
from ftmoe.kernel._dequant import dequant

pytestmark = pytest.mark.gpu


def _eq(got: torch.Tensor, ref: np.ndarray, what: str):
    g = got.float().cpu().numpy()
    nan_ok = np.array_equal(np.isnan(g), np.isnan(ref))
    assert nan_ok, f"{what}: NaN positions differ"
    m = ~np.isnan(ref)
    bad = g[m] != ref[m]
    assert not bad.any(), f"{what}: {int(bad.sum())} mismatches, first got {g[m][bad][:4]} ref {ref[m][bad][:4]}"


def _round(ref_f32: np.ndarray, dt: torch.dtype) -> np.ndarray:
    if dt == torch.bfloat16:
        return O.round_bf16(ref_f32)
    if dt == torch.float16:
        return ref_f32.astype(np.float16).astype(np.float32)
    return ref_f32


def _fp8_all_codes(gpu):
    w = torch.arange(256, dtype=torch.uint8).repeat(64, 2)  # [64, 512], every code 2x per row
    w = w.view(torch.float8_e4m3fn)
    s = torch.tensor([[1.0, 0.3711, 2.0 ** -10, 7.5e-3]], dtype=torch.float32)
    return w, s


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fp8_dequant_all_codes(gpu, out_dtype):
    w, s = _fp8_all_codes(gpu)
    ref = O.dequantize_block_fp8(np_(w), s.numpy(), 128)
    got = dequant(single_proj("fp8_block", w.to(gpu), 64, 512, s=s.to(gpu), group=128), out_dtype=out_dtype)
    _eq(got, _round(ref, out_dtype), f"fp8 dequant {out_dtype}")


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_mxfp4_dequant_all_bytes_and_edge_exponents(gpu, out_dtype):
    blocks = torch.arange(256, dtype=torch.uint8).reshape(16, 16).repeat(16, 1).reshape(16, 16, 16)  # [16 rows, 16 blocks, 16]
    scales = torch.tensor([0, 1, 2, 100, 120, 126, 127, 128, 140, 200, 250, 253, 254, 255, 127, 127],
                          dtype=torch.uint8).repeat(16, 1)  # [16, 16]
    ref = O.dequantize_mxfp4_blocks(blocks.numpy(), scales.numpy())
    got = dequant(single_proj("mxfp4", blocks.to(gpu), 16, 512, s=scales.to(gpu), group=32), out_dtype=out_dtype)
    _eq(got, _round(ref, out_dtype), f"mxfp4 dequant {out_dtype}")


def test_gptq_dequant_random(gpu):
    from ftmoe import quant

    g = torch.Generator().manual_seed(0)
    w = torch.randn(512, 384, generator=g)  # [K, N]
    qw, qz, sc = quant.quantize_gptq_int4(w, group_size=128)
    qw, qz = qw.clone(), qz.clone()
    qz ^= torch.randint(0, 2 ** 31 - 1, qz.shape, generator=g, dtype=torch.int32) & 0x33333333  # varied zeros
    ref = O.dequantize_gptq_int4(qw.numpy(), qz.numpy(), sc.numpy(), 128)  # [K, N]
    proj = single_proj("gptq_int4", qw.to(gpu), 384, 512, s=sc.to(gpu), z=qz.to(gpu), group=128)
    _eq(dequant(proj, out_dtype=torch.float32, transpose=True), ref, "gptq dequant [K,N]")
    _eq(dequant(proj, out_dtype=torch.bfloat16, transpose=False), O.round_bf16(ref.T.copy()), "gptq dequant [N,K] bf16")


@pytest.mark.parametrize("num_groups", [1, 4, 8])
def test_int8_dequant_random(gpu, num_groups):
    g = torch.Generator().manual_seed(1)
    codes = torch.randint(-128, 128, (96, 256), generator=g, dtype=torch.int16).to(torch.int8)
    from ftmoe import quant

    wp = quant.pack_int8_to_int32(codes)
    s = torch.rand(96, num_groups, generator=g) * 0.1 + 0.01
    ref = O.dequantize_int8_packed(wp.numpy(), s.numpy(), 256)
    got = dequant(single_proj("int8_channel", wp.to(gpu), 96, 256, s=s.to(gpu), group=256 // num_groups),
                  out_dtype=torch.float32)
    _eq(got, ref, "int8 dequant")
    s16 = s.to(torch.bfloat16)
    ref16 = O.dequantize_int8_packed(wp.numpy(), O.bf16_bits_to_f32(np_(s16)), 256)
    got16 = dequant(single_proj("int8_channel", wp.to(gpu), 96, 256, s=s16.to(gpu), group=256 // num_groups),
                    out_dtype=torch.bfloat16)
    _eq(got16, O.round_bf16(ref16), "int8 dequant bf16 scales")


# ---------------------------------------------------------------- register decode through the MFMA engine
def _identity_check(gpu, proj, ref_nk: np.ndarray, what: str):
    K = proj.K
    eye = torch.eye(K, dtype=torch.float32, device=gpu)
    got = run_linear(proj, eye, out_dtype=torch.float32, bias=None)  # [K, N] = W^T
    _eq(got, np.ascontiguousarray(ref_nk.T), what)


def test_fp8_register_decode_exact(gpu):
    w, s = _fp8_all_codes(gpu)
    wc = w.view(torch.uint8).clone()
    wc[(wc & 0x7F) == 0x7F] = 0x3C  # the MFMA path is not defined for NaN weights
    w = wc.view(torch.float8_e4m3fn)
    ref = O.dequantize_block_fp8(np_(w), s.numpy(), 128)
    _identity_check(gpu, single_proj("fp8_block", w.to(gpu), 64, 512, s=s.to(gpu), group=128), ref, "fp8 mfma decode")


def test_mxfp4_register_decode_exact(gpu):
    blocks = torch.arange(256, dtype=torch.uint8).reshape(16, 16).repeat(16, 1).reshape(16, 16, 16)
    scales = torch.tensor([2, 3, 100, 120, 126, 127, 128, 140, 200, 250, 230, 240, 120, 122, 127, 130],
                          dtype=torch.uint8).repeat(16, 1)
    ref = O.dequantize_mxfp4_blocks(blocks.numpy(), scales.numpy())
    _identity_check(gpu, single_proj("mxfp4", blocks.to(gpu), 16, 512, s=scales.to(gpu), group=32), ref,
                    "mxfp4 mfma decode")


def test_gptq_register_decode_exact(gpu):
    from ftmoe import quant

    g = torch.Generator().manual_seed(2)
    qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (512 // 8, 128), generator=g, dtype=torch.int64).to(torch.int32)
    qz = torch.randint(-2 ** 31, 2 ** 31 - 1, (4, 128 // 8), generator=g, dtype=torch.int64).to(torch.int32)
    sc = (torch.rand(4, 128, generator=g) * 0.01 + 1e-3).to(torch.float16)
    ref = O.dequantize_gptq_int4(qw.numpy(), qz.numpy(), sc.numpy(), 128).T  # [N, K]
    proj = single_proj("gptq_int4", qw.to(gpu), 128, 512, s=sc.to(gpu), z=qz.to(gpu), group=128)
    _identity_check(gpu, proj, ref, "gptq mfma decode")
    del quant


@pytest.mark.parametrize("num_groups", [1, 2])
def test_int8_register_decode_exact(gpu, num_groups):
    from ftmoe import quant

    g = torch.Generator().manual_seed(3)
    codes = torch.randint(-128, 128, (64, 256), generator=g, dtype=torch.int16).to(torch.int8)
    wp = quant.pack_int8_to_int32(codes)
    s = torch.rand(64, num_groups, generator=g) * 0.1 + 0.01
    ref = O.dequantize_int8_packed(wp.numpy(), s.numpy(), 256)
    _identity_check(gpu, single_proj("int8_channel", wp.to(gpu), 64, 256, s=s.to(gpu), group=256 // num_groups),
                    ref, "int8 mfma decode")


def test_bf16_identity_exact(gpu):
    g = torch.Generator().manual_seed(4)
    w = torch.randn(48, 256, generator=g).to(torch.bfloat16)
    _identity_check(gpu, single_proj("bf16", w.to(gpu), 48, 256), O.bf16_bits_to_f32(np_(w)), "bf16 mfma")
