"""GPU: the per-projection drop-in API (fused_{fp8,gptq,int8,mxfp4}_linear and
*_expert_forward) against the oracle's dequantize-then-matmul, at the shapes
and tolerances of the reference's own tests
(tests/test_fused_fp8_linear_xpu.py:24-46, test_gptq_fused_linear_xpu.py,
test_fused_int8_linear_xpu.py:39-64, test_fused_mxfp4_linear_xpu.py), plus
their bias / out_dtype / error-message checks."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import np_

from ftmoe import quant
from ftmoe.kernel.fused_fp8_linear import fused_fp8_expert_forward, fused_fp8_linear
from ftmoe.kernel.fp8_block_linear import dequantize_block_fp8
from ftmoe.kernel.fused_int8_linear import fused_int8_expert_forward, fused_int8_linear
from ftmoe.kernel.fused_mxfp4_linear import fused_mxfp4_expert_forward, fused_mxfp4_linear
from ftmoe.kernel.gptq_fused_linear import fused_gptq_expert_forward, fused_gptq_linear

pytestmark = pytest.mark.gpu


def _check(got, x, w_nk, atol, rtol, bias=None):
    ref = x.double().cpu().numpy() @ w_nk.astype(np.float64).T
    if bias is not None:
        ref = ref + bias.double().cpu().numpy()
    np.testing.assert_allclose(got.double().cpu().numpy(), ref, atol=atol, rtol=rtol)


@pytest.mark.parametrize("m,k,n,block", [(8, 256, 384, 128), (5, 300, 213, 128), (32, 2048, 768, 128),
                                         (1, 128, 128, 128), (64, 2048, 1024, 128)])
def test_fp8_matches_dequant_then_matmul(gpu, m, k, n, block):
    g = torch.Generator().manual_seed(0)
    w = torch.randn(n, k, generator=g)
    wq, s = quant.quantize_block_fp8(w, block=block)
    x = torch.randn(m, k, generator=g)
    got = fused_fp8_linear(x.to(gpu), wq.to(gpu), s.to(gpu), block=block, out_dtype=torch.float32)
    _check(got, x, O.dequantize_block_fp8(np_(wq), s.numpy(), block), 2e-3, 2e-2)


def test_fp8_bias_dtype_and_errors(gpu):
    g = torch.Generator().manual_seed(1)
    w = torch.randn(32, 128, generator=g)
    wq, s = quant.quantize_block_fp8(w)
    x = torch.randn(4, 128, generator=g)
    bias = torch.randn(32, generator=g)
    got = fused_fp8_linear(x.to(gpu), wq.to(gpu), s.to(gpu), bias=bias.to(gpu), out_dtype=torch.float32)
    _check(got, x, O.dequantize_block_fp8(np_(wq), s.numpy()), 2e-3, 2e-2, bias=bias)
    assert fused_fp8_linear(x.to(gpu, torch.bfloat16), wq.to(gpu), s.to(gpu)).dtype == torch.bfloat16
    with pytest.raises(ValueError, match="must divide"):
        fused_fp8_linear(x.to(gpu), wq.to(gpu), s.to(gpu), block_n=24)
    with pytest.raises(TypeError, match="fp8"):
        fused_fp8_linear(x.to(gpu), w.to(gpu), s.to(gpu))
    with pytest.raises(ValueError, match="does not match"):
        fused_fp8_linear(x.to(gpu), wq.to(gpu), s[:, :0].to(gpu))


@pytest.mark.parametrize("m,k,n,group", [(1, 2048, 768, 128), (4, 256, 128, 128), (32, 2048, 768, 128),
                                         (7, 384, 264, 128), (3, 256, 64, 32)])
def test_gptq_matches_dequant_then_matmul(gpu, m, k, n, group):
    g = torch.Generator().manual_seed(2)
    w = torch.randn(k, n, generator=g)
    qw, qz, sc = quant.quantize_gptq_int4(w, group_size=group)
    x = torch.randn(m, k, generator=g)
    got = fused_gptq_linear(x.to(gpu), qw.to(gpu), qz.to(gpu), sc.to(gpu), group_size=group, out_dtype=torch.float32)
    _check(got, x, O.dequantize_gptq_int4(qw.numpy(), qz.numpy(), sc.numpy(), group).T, 1e-3, 1e-3)


def _pack_int8(codes):  # tests/test_fused_int8_linear_xpu.py:26-31 convention
    return quant.pack_int8_to_int32(codes)


@pytest.mark.parametrize("m,k,n,group", [(8, 64, 32, 32), (5, 384, 504, 128), (32, 2048, 768, 128),
                                         (4, 1024, 1024, 1024)])
def test_int8_matches_dequant_then_matmul(gpu, m, k, n, group):
    g = torch.Generator().manual_seed(100 + k)
    codes = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    scale = torch.rand(n, k // group, generator=g) * 0.1 + 0.01
    wp = _pack_int8(codes)
    x = torch.randn(m, k, generator=g)
    got = fused_int8_linear(x.to(gpu), wp.to(gpu), scale.to(gpu), k=k, out_dtype=torch.float32)
    _check(got, x, O.dequantize_int8_packed(wp.numpy(), scale.numpy(), k), 2e-3, 2e-2)


def test_int8_errors(gpu):
    wp = torch.zeros(8, 4, dtype=torch.int32, device=gpu)
    x = torch.zeros(2, 16, device=gpu)
    with pytest.raises(ValueError, match="below the fused kernel's minimum"):
        fused_int8_linear(x, wp, torch.ones(8, 4, device=gpu), k=16)
    with pytest.raises(ValueError, match="not evenly divisible"):
        fused_int8_linear(x, wp, torch.ones(8, 3, device=gpu), k=16)
    with pytest.raises(TypeError, match="int32"):
        fused_int8_linear(x, wp.float(), torch.ones(8, 1, device=gpu), k=16)


@pytest.mark.parametrize("m,k,n", [(8, 64, 32), (5, 96, 40), (32, 2048, 768), (1, 2880, 5760)])
def test_mxfp4_matches_dequant_then_matmul(gpu, m, k, n):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(n, k, generator=g) * 0.5
    blocks, scales = quant.quantize_mxfp4_blocks(w)
    x = torch.randn(m, k, generator=g)
    got = fused_mxfp4_linear(x.to(gpu), blocks.to(gpu), scales.to(gpu), out_dtype=torch.float32)
    _check(got, x, O.dequantize_mxfp4_blocks(blocks.numpy(), scales.numpy()), 2e-3, 2e-2)


def test_mxfp4_errors(gpu):
    with pytest.raises(TypeError, match="uint8"):
        fused_mxfp4_linear(torch.zeros(1, 32, device=gpu), torch.zeros(4, 1, 16, dtype=torch.int32, device=gpu),
                           torch.zeros(4, 1, dtype=torch.uint8, device=gpu))
    with pytest.raises(ValueError, match="16 packed bytes"):
        fused_mxfp4_linear(torch.zeros(1, 32, device=gpu), torch.zeros(4, 1, 8, dtype=torch.uint8, device=gpu),
                           torch.zeros(4, 1, dtype=torch.uint8, device=gpu))


def _expert_ref(x, gu_nk, dn_nk, inter, h_dt="bf16"):
    """gu in float64, h = silu(g) * u rounded to ``h_dt`` (the reference rounds h
    to out_dtype, fused_fp8_linear.py:174), y = h . W2^T in float64."""
    gu = x.double().numpy() @ gu_nk.astype(np.float64).T
    g, u = gu[:, :inter], gu[:, inter:]
    h = O.act("silu", g, u)
    h = O.round_to(h.astype(np.float32), h_dt).astype(np.float64)
    return h @ dn_nk.astype(np.float64).T


def test_fp8_expert_forward(gpu):
    g = torch.Generator().manual_seed(4)
    I, H = 256, 512
    gu = torch.randn(2 * I, H, generator=g) * 0.02
    dn = torch.randn(H, I, generator=g) * 0.02
    qg, sg = quant.quantize_block_fp8(gu)
    qd, sd = quant.quantize_block_fp8(dn)
    x = torch.randn(3, H, generator=g).to(torch.bfloat16)
    got = fused_fp8_expert_forward(x.to(gpu), qg.to(gpu), sg.to(gpu), qd.to(gpu), sd.to(gpu), intermediate=I)
    assert got.dtype == torch.bfloat16
    ref = _expert_ref(x.float(), O.dequantize_block_fp8(np_(qg), sg.numpy()), O.dequantize_block_fp8(np_(qd), sd.numpy()), I)
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


def test_gptq_expert_forward(gpu):
    g = torch.Generator().manual_seed(5)
    I, H = 256, 512
    gu = torch.randn(H, 2 * I, generator=g) * 0.02  # [K, N]
    dn = torch.randn(I, H, generator=g) * 0.02
    a = quant.quantize_gptq_int4(gu)
    b = quant.quantize_gptq_int4(dn)
    x = torch.randn(5, H, generator=g).to(torch.bfloat16)
    got = fused_gptq_expert_forward(x.to(gpu), *[t.to(gpu) for t in a], *[t.to(gpu) for t in b], group_size=128,
                                    intermediate=I)
    ref = _expert_ref(x.float(), O.dequantize_gptq_int4(*[t.numpy() for t in a], 128).T,
                      O.dequantize_gptq_int4(*[t.numpy() for t in b], 128).T, I)
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


_DT_NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("xdt,odt", [(torch.float16, None), (torch.bfloat16, torch.float16),
                                     (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
def test_fp8_expert_forward_rounds_h_to_out_dtype(gpu, xdt, odt):
    """h is rounded to out_dtype (default x.dtype) between the projections, as
    the reference's two fused calls do (fused_fp8_linear.py:172-175): fp16 h
    for fp16 inputs, whatever the activations' dtype.  The check is tight
    enough to tell an fp16 from a bf16 rounding of h."""
    g = torch.Generator().manual_seed(44)
    I, H = 256, 512
    gu = torch.randn(2 * I, H, generator=g) * 0.05
    dn = torch.randn(H, I, generator=g) * 0.05
    qg, sg = quant.quantize_block_fp8(gu)
    qd, sd = quant.quantize_block_fp8(dn)
    x = torch.randn(6, H, generator=g).to(xdt)
    out_dt = odt if odt is not None else xdt
    got = fused_fp8_expert_forward(x.to(gpu), qg.to(gpu), sg.to(gpu), qd.to(gpu), sd.to(gpu), intermediate=I,
                                   out_dtype=odt)
    assert got.dtype == out_dt
    Wg, Wd = O.dequantize_block_fp8(np_(qg), sg.numpy()), O.dequantize_block_fp8(np_(qd), sd.numpy())
    ref = _expert_ref(x.float(), Wg, Wd, I, h_dt=_DT_NAME[out_dt])
    ref = O.round_to(ref.astype(np.float32), _DT_NAME[out_dt]).astype(np.float64)
    err = np.abs(got.double().cpu().numpy() - ref).max()
    scale = np.abs(ref).max()
    # fp32 x keeps ~16 bits through the bf16 hi + lo split: allow that, plus one output ulp
    tol = {"f32": 2e-4, "f16": 7e-4, "bf16": 8e-3}[_DT_NAME[out_dt]] * scale
    assert err <= tol, (err, tol)
    if out_dt != torch.bfloat16:  # the other rounding of h is outside that bound
        alt = _expert_ref(x.float(), Wg, Wd, I, h_dt="bf16")
        assert np.abs(alt - ref).max() > tol


@pytest.mark.parametrize("M", [1, 3, 70])
def test_int8_expert_forward(gpu, M):
    """fused_int8_expert_forward (fused_int8_linear.py:176-201) on per-channel
    banks: the decode stages at 1 and 3 rows, the tiled stages above the
    crossover."""
    g = torch.Generator().manual_seed(6 + M)
    I, H = 256, 512
    cg = torch.randint(-127, 128, (2 * I, H), generator=g, dtype=torch.int8)
    cd = torch.randint(-127, 128, (H, I), generator=g, dtype=torch.int8)
    sg = torch.rand(2 * I, 1, generator=g) * 1e-3 + 1e-4
    sd = torch.rand(H, 1, generator=g) * 1e-3 + 1e-4
    wg, wd = _pack_int8(cg), _pack_int8(cd)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    got = fused_int8_expert_forward(x.to(gpu), wg.to(gpu), sg.to(gpu), wd.to(gpu), sd.to(gpu), intermediate=I,
                                    k_gate_up=H, k_down=I)
    assert got.dtype == torch.bfloat16
    ref = _expert_ref(x.float(), O.dequantize_int8_packed(wg.numpy(), sg.numpy(), H),
                      O.dequantize_int8_packed(wd.numpy(), sd.numpy(), I), I)
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("M", [1, 4, 130])
def test_mxfp4_expert_forward(gpu, M):
    """fused_mxfp4_expert_forward (fused_mxfp4_linear.py:191-210): SiLU SwiGLU
    over MXFP4 banks at a gpt-oss-like width."""
    g = torch.Generator().manual_seed(8 + M)
    I, H = 320, 640
    bg, eg = quant.quantize_mxfp4_blocks(torch.randn(2 * I, H, generator=g) * 0.05)
    bd, ed = quant.quantize_mxfp4_blocks(torch.randn(H, I, generator=g) * 0.05)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    got = fused_mxfp4_expert_forward(x.to(gpu), bg.to(gpu), eg.to(gpu), bd.to(gpu), ed.to(gpu), intermediate=I)
    ref = _expert_ref(x.float(), O.dequantize_mxfp4_blocks(bg.numpy(), eg.numpy()),
                      O.dequantize_mxfp4_blocks(bd.numpy(), ed.numpy()), I)
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


def test_e5m2_dequant_every_code(gpu):
    """float8_e5m2 weights (accepted by fused_fp8_linear, fused_fp8_linear.py:123):
    every one of the 256 codes through the dequant kernel equals torch's own
    e5m2 -> fp32 conversion times the block scale (inf and NaN included)."""
    codes = torch.arange(256, dtype=torch.uint8).reshape(2, 128)
    w = codes.view(torch.float8_e5m2)
    s = torch.tensor([[0.5]], dtype=torch.float32)
    got = dequantize_block_fp8(w.to(gpu), s.to(gpu), out_dtype=torch.float32).cpu()
    want = w.float() * 0.5
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    fin = ~torch.isnan(want)
    assert torch.equal(got[fin], want[fin])


@pytest.mark.parametrize("m,k,n", [(3, 256, 200), (9, 384, 256)])
def test_fp8_e5m2_linear_matches_dequant_then_matmul(gpu, m, k, n):
    g = torch.Generator().manual_seed(9)
    w = (torch.randn(n, k, generator=g) * 0.1).to(torch.float8_e5m2)
    s = torch.rand(-(-n // 128), -(-k // 128), generator=g) + 0.5
    x = torch.randn(m, k, generator=g)
    got = fused_fp8_linear(x.to(gpu), w.to(gpu), s.to(gpu), out_dtype=torch.float32)
    # the reference's dequant (fp8_block_linear.py:48-91): fp32(w) times its block's scale
    dense = w.float() * torch.repeat_interleave(torch.repeat_interleave(s, 128, 0), 128, 1)[:n, :k]
    _check(got, x, dense.numpy(), 2e-3, 2e-2)
