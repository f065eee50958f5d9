"""CPU: the two-term e4m3 split of the input that the MXFP4 decode stage
feeds to the scaled fp8 x fp4 MFMAs (k_quant_mx in ftm_moe.hip), restated
here and pinned by what the arithmetic fixes: hi * s_hi + lo * s_lo is the
bf16 input itself for every element within 2^-13 of its block's maximum and
off by at most 2^(E - 21) below that; codes stay finite (no 0x7f / 0xff
e4m3, scales <= 247); and the GPU test's relative-error bound separates the
split from the one-term rounding it replaces (the mistake planted in the
oracle's input)."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import MX_REL_RMS, np_, oracle_spec, rel_rms, wide_range_x

from ftmoe import synthetic as S


def mx_split(x: torch.Tensor):
    """x bf16 [T, H] (H % 32 == 0) -> (hi, lo) e4m3 [T, H/32, 32] and their
    e8m0 codes [T, H/32]: E = floor(log2 max|x|) per block, s_hi = 2^(E - 7)
    (code E + 120 clamped to >= 0), s_lo = s_hi / 16."""
    T, H = x.shape
    xb = x.float().reshape(T, H // 32, 32)
    amax = xb.abs().amax(-1)
    ebits = (amax.view(torch.int32) >> 23) & 0xFF
    chi = (ebits - 7).clamp(min=0)
    clo = (chi - 4).clamp(min=0)
    s_hi = torch.exp2((chi - 127).double()).unsqueeze(-1)
    s_lo = torch.exp2((clo - 127).double()).unsqueeze(-1)
    v = (xb.double() / s_hi).float()
    hi = v.to(torch.float8_e4m3fn)
    r = ((v.double() - hi.double()) * (s_hi / s_lo)).float()
    lo = r.to(torch.float8_e4m3fn)
    return hi, lo, chi, clo, s_hi, s_lo


def test_split_reconstructs_bf16_inputs():
    g = torch.Generator().manual_seed(7)
    T, H = 64, 2880
    # per-block exponents from tiny to huge, per-element spread of 2^-20 .. 1 inside a block
    be = torch.randint(-110, 120, (T, H // 32, 1), generator=g).float()
    ee = torch.randint(-20, 1, (T, H // 32, 32), generator=g).float()
    x = (torch.randn(T, H // 32, 32, generator=g) * torch.exp2(be + ee)).reshape(T, H).to(torch.bfloat16)
    x[0, :32] = 0  # an all-zero block
    hi, lo, chi, clo, s_hi, s_lo = mx_split(x)
    xr = hi.double() * s_hi + lo.double() * s_lo
    xd = x.double().reshape(T, H // 32, 32)
    E = (chi + 120 - 127).double().unsqueeze(-1)  # floor(log2 amax) where unclamped
    big = xd.abs() >= torch.exp2(E - 13)
    assert torch.equal(xr[big], xd[big])
    assert (xr - xd).abs().le(torch.exp2(E - 21)).all()
    for q in (hi, lo):
        c = q.view(torch.uint8) & 0x7F
        assert int(c.max()) < 0x7F
    assert int(chi.max()) <= 247 and int(clo.min()) >= 0
    assert torch.all(xr[0, 0] == 0)


def test_split_magnitudes_fit_e4m3():
    """|x / s_hi| < 256 and the residual term |r * 16| <= 128: far inside the
    e4m3 range (448), so no value saturates."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(16, 4096, generator=g) * 1e3).to(torch.bfloat16)
    hi, lo, *_ = mx_split(x)
    assert hi.float().abs().max() <= 256 and lo.float().abs().max() <= 128


@pytest.mark.parametrize("T", [4, 32])
def test_rel_rms_bound_separates_split_from_one_term(T):
    syn = S.generate(S.SMALL["c4_mxfp4"], T=T, seed=21)
    spec = oracle_spec(syn)
    x = wide_range_x(T, syn.cfg.H, seed=T)
    ref = O.layer_reference(spec, np_(x))["out"]
    hi, lo, _, _, s_hi, s_lo = mx_split(x)
    one = (hi.double() * s_hi).reshape(T, -1).to(torch.bfloat16)  # planted: the lo term dropped
    two = (hi.double() * s_hi + lo.double() * s_lo).reshape(T, -1).to(torch.bfloat16)
    assert torch.equal(two.view(torch.int16), x.view(torch.int16)) or \
        rel_rms(two.float().numpy(), x.float().numpy()) < 1e-5
    err_one = rel_rms(O.layer_reference(spec, np_(one))["out"], ref)
    assert err_one > 2 * MX_REL_RMS, err_one
