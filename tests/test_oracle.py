"""Pins of the CPU oracle (oracle/) -- CPU only.

Each check is chosen so a plausible slip in the restatement (wrong nibble
order, dropped +1 on the GPTQ zero point, wrong exponent bias, transposed
operand, wrong tie order) fails it:
  * the reference's own known-answer tests, re-expressed as fixtures
    (tests/test_gptq_quant.py:31-69, tests/test_weight_gptq_banks.py:90-111,
    tests/test_mxfp4_quant.py:23-46,86-90);
  * OCP e4m3 / e8m0 closed forms against torch's float8 dtypes (a library);
  * the numpy and C restatements of every dequant against each other;
  * routing against torch softmax/topk and hand-computed tie cases;
  * the layer against an independent float64 brute force and against the
    reference's own CPU MoE kernel (cpu_moe.cpp, built unmodified into oracle/_ref).
"""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import np_, oracle_spec


def _pack_nibbles(codes):
    word = 0
    for i, c in enumerate(codes):
        word |= c << (4 * i)
    return np.uint32(word).view(np.int32)


# ------------------------------------------------------------------ GPTQ
def test_gptq_known_encoding_codes_0_to_7():
    # tests/test_gptq_quant.py:31-50: codes 0..7 down K, zero nibble 7 (zero 8), scale 0.5
    qweight = np.full((1, 8), _pack_nibbles(list(range(8))), np.int32)
    qzeros = np.array([[_pack_nibbles([7] * 8)]], np.int32)
    scales = np.full((1, 8), 0.5, np.float32)
    out = O.dequantize_gptq_int4(qweight, qzeros, scales, 8)
    expected = np.array([0.5 * (c - 8) for c in range(8)], np.float32)
    for n in range(8):
        np.testing.assert_array_equal(out[:, n], expected)
    p = O.OracleProj("gptq_int4", qweight, 8, 8, s=scales.astype(np.float16), z=qzeros, group=8)
    np.testing.assert_array_equal(O.dequant(p).T, out)


def test_gptq_per_group_scale_and_zero():
    # tests/test_gptq_quant.py:53-69: group 0 -> 1*(1-8) = -7, group 1 -> 10*(1-4) = -30
    qweight = np.full((1, 8), _pack_nibbles([1] * 8), np.int32)
    qzeros = np.array([[_pack_nibbles([7] * 8)], [_pack_nibbles([3] * 8)]], np.int32)
    scales = np.array([[1.0] * 8, [10.0] * 8], np.float32)
    out = O.dequantize_gptq_int4(qweight, qzeros, scales, 4)
    np.testing.assert_array_equal(out[:4, 0], np.full(4, -7.0, np.float32))
    np.testing.assert_array_equal(out[4:, 0], np.full(4, -30.0, np.float32))
    p = O.OracleProj("gptq_int4", qweight, 8, 8, s=scales, z=qzeros, group=4)
    np.testing.assert_array_equal(O.dequant(p).T, out)


def test_gptq_bank_fixture_value():
    # tests/test_weight_gptq_banks.py:90-111: code 5, zero nibble 7, scale 0.5 -> -1.5
    k, n, g = 16, 8, 8
    qweight = np.full((k // 8, n), _pack_nibbles([5] * 8), np.int32)
    qzeros = np.full((k // g, n // 8), _pack_nibbles([7] * 8), np.int32)
    scales = np.full((k // g, n), 0.5, np.float16)
    np.testing.assert_array_equal(O.dequantize_gptq_int4(qweight, qzeros, scales, g), np.full((k, n), -1.5))


def test_gptq_nibble_order_is_lsb_first():
    # a word holding codes 0..7 must give code i at row i (not 7-i)
    qweight = np.array([[_pack_nibbles([3, 0, 0, 0, 0, 0, 0, 9])]], np.int32)
    qzeros = np.array([[_pack_nibbles([0] * 8)]], np.int32)  # zero point 1
    out = O.dequantize_gptq_int4(np.repeat(qweight, 8, axis=1), np.repeat(qzeros, 1, axis=1),
                                 np.ones((1, 8), np.float32), 8)
    assert out[0, 0] == 2.0 and out[7, 0] == 8.0 and out[1, 0] == -1.0


# ------------------------------------------------------------------ MXFP4
def test_mxfp4_known_encoding():
    # tests/test_mxfp4_quant.py:23-36
    block = np.zeros((1, 16), np.uint8)
    block[0, 0], block[0, 1] = 0x10, 0x32
    out = O.dequantize_mxfp4_blocks(block, np.array([127], np.uint8))
    expected = np.zeros(32, np.float32)
    expected[:4] = [0.0, 0.5, 1.0, 1.5]
    np.testing.assert_array_equal(out, expected)  # [1 block, 16] -> [32]


def test_mxfp4_scale_is_power_of_two():
    # tests/test_mxfp4_quant.py:39-46: e8m0 128 doubles
    block = np.zeros((1, 16), np.uint8)
    block[0, 0] = 0x02
    assert O.dequantize_mxfp4_blocks(block, np.array([128], np.uint8))[0] == 2.0


def test_mxfp4_all_zero_block_round_trips():
    # tests/test_mxfp4_quant.py:86-90
    b, s = O.quantize_mxfp4_blocks(np.zeros((1, 32), np.float32))
    np.testing.assert_array_equal(O.dequantize_mxfp4_blocks(b, s), np.zeros((1, 32), np.float32))


def test_e8m0_edges_match_torch_exp2():
    s = np.arange(256)
    ref = torch.exp2(torch.tensor(s, dtype=torch.float32) - 127).numpy()
    np.testing.assert_array_equal(O.e8m0_to_f32(s), ref)


def test_mxfp4_lut_matches_torch_float4_e2m1():
    # every nibble through torch's own e2m1 dtype (low nibble first)
    codes = torch.arange(16, dtype=torch.uint8) | (torch.arange(16, dtype=torch.uint8) << 4)
    if not hasattr(torch, "float4_e2m1fn_x2"):
        pytest.skip("torch has no float4_e2m1fn_x2")
    try:
        vals = codes.view(torch.float4_e2m1fn_x2).to(torch.float32)
    except (RuntimeError, NotImplementedError):
        pytest.skip("torch cannot convert float4_e2m1fn_x2 on this build")
    np.testing.assert_array_equal(vals.numpy().reshape(-1)[0::2], O.E2M1)


def test_mxfp4_c_matches_numpy():
    rng = np.random.RandomState(3)
    blocks = rng.randint(0, 256, size=(2, 24, 4, 16)).astype(np.uint8)
    scales = rng.randint(100, 140, size=(2, 24, 4)).astype(np.uint8)
    p = O.OracleProj("mxfp4", blocks, 24, 128, s=scales, group=32)
    for slot in range(2):
        np.testing.assert_array_equal(O.dequant(p, slot), O.dequantize_mxfp4_blocks(blocks[slot], scales[slot]))


# ------------------------------------------------------------------ FP8
def test_e4m3_lut_matches_torch_all_codes():
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    np.testing.assert_array_equal(np.isnan(t), np.isnan(O.E4M3))
    np.testing.assert_array_equal(np.nan_to_num(t), np.nan_to_num(O.E4M3))
    # the C decode agrees too
    c = np.array([O.lib().orc_e4m3_to_f32(b) for b in range(256)], np.float32)
    np.testing.assert_array_equal(np.nan_to_num(c), np.nan_to_num(O.E4M3))


def test_e4m3_encode_matches_torch_cast():
    rng = np.random.RandomState(0)
    fin = O.E4M3[~np.isnan(O.E4M3)]
    mids = ((O.E4M3[1:127].astype(np.float64) + O.E4M3[:126]) / 2).astype(np.float32)
    x = np.concatenate([rng.randn(100000).astype(np.float32) * 40, fin, mids, -mids,
                        np.array([448, 464, 465, 1e-9, -1e-9, 0.0, -0.0], np.float32)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.f32_to_e4m3(x), ref)


def test_fp8_dequant_closed_form_and_c_agree():
    rng = np.random.RandomState(1)
    N, K, B = 200, 384, 128
    w = rng.randint(0, 256, size=(N, K)).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x11  # no NaN codes
    s = (rng.rand(2, 3).astype(np.float32) * 1e-3)
    ref = (torch.from_numpy(w).view(torch.float8_e4m3fn).to(torch.float32)
           * torch.from_numpy(s).repeat_interleave(B, 0)[:N].repeat_interleave(B, 1)[:, :K]).numpy()
    np.testing.assert_array_equal(O.dequantize_block_fp8(w, s, B), ref)
    np.testing.assert_array_equal(O.dequant(O.OracleProj("fp8_block", w, N, K, s=s, group=B)), ref)


# ------------------------------------------------------------------ INT8
def test_int8_pack_known_bytes():
    # offset-binary: stored byte = value + 128, byte 0 = lowest k (int8_packed_linear.py:26-38)
    codes = np.array([[-128, -1, 0, 127]], np.int8)
    word = O.pack_int8(codes)
    assert word.view(np.uint32)[0, 0] == 0xFF807F00
    out = O.dequantize_int8_packed(word, np.ones((1, 1), np.float32), 4)
    np.testing.assert_array_equal(out, codes.astype(np.float32))


def test_int8_grouped_c_matches_numpy():
    rng = np.random.RandomState(2)
    codes = rng.randint(-127, 128, size=(3, 40, 256)).astype(np.int8)
    wp = O.pack_int8(codes)
    s = (rng.rand(3, 40, 4) * 0.1 + 0.01).astype(np.float32)
    p = O.OracleProj("int8_channel", wp, 40, 256, s=s, group=64)
    for slot in range(3):
        ref = codes[slot].astype(np.float32) * np.repeat(s[slot], 64, axis=1)
        np.testing.assert_array_equal(O.dequantize_int8_packed(wp[slot], s[slot], 256), ref)
        np.testing.assert_array_equal(O.dequant(p, slot), ref)


# ------------------------------------------------------------------ routing
def test_router_logits_within_one_bf16_ulp_of_torch_linear():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(9, 512, generator=g).to(torch.bfloat16)
    G = (torch.randn(40, 512, generator=g) * 0.02).to(torch.bfloat16)
    ref = torch.nn.functional.linear(x, G).float().numpy()
    got = O.router_logits(np_(x), np_(G))
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)


def test_router_logits_are_an_exact_fp32_dot_order():
    # the fixed GPU order sums to the double-precision dot up to fp32 rounding
    rng = np.random.RandomState(5)
    x = O.f32_to_bf16_bits(rng.randn(3, 2048).astype(np.float32))
    G = O.f32_to_bf16_bits((rng.randn(7, 2048) * 0.02).astype(np.float32))
    got = O.router_logits(x, G)
    ref = O.bf16_bits_to_f32(x).astype(np.float64) @ O.bf16_bits_to_f32(G).astype(np.float64).T
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)


def test_route_tie_breaks_to_lower_index_and_renorms():
    logits = np.array([[1.0, 3.0, 2.0, 3.0]], np.float32)
    ids, w = O.route(logits, 2, "softmax_topk", True, weight_dt="f32")
    assert ids.tolist() == [[1, 3]]
    np.testing.assert_allclose(w, [[0.5, 0.5]], rtol=1e-7)
    ids, w = O.route(logits, 3, "topk_softmax", True, weight_dt="f32")
    assert ids.tolist() == [[1, 3, 2]]
    e = np.exp(np.array([0.0, 0.0, -1.0]))
    np.testing.assert_allclose(w[0], e / e.sum(), rtol=1e-6)


def test_route_matches_torch_softmax_topk():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(64, 256, generator=g).to(torch.bfloat16).float()
    p = torch.softmax(logits, dim=-1, dtype=torch.float32)
    tw, ti = torch.topk(p, 8, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).to(torch.bfloat16).float()
    ids, w = O.route(logits.numpy(), 8, "softmax_topk", True)
    # compare rows without ties among the top 9 (torch's tie order is unspecified)
    srt = np.sort(logits.numpy(), axis=1)[:, ::-1]
    ok = srt[:, 7] > srt[:, 8]
    assert ok.sum() > 40
    for t in np.nonzero(ok)[0]:
        assert sorted(ids[t].tolist()) == sorted(ti[t].tolist())
    np.testing.assert_allclose(np.sort(w[ok], 1), np.sort(tw.numpy()[ok], 1), rtol=2 ** -7)


def _tie_free_rows(keys: np.ndarray, k: int) -> np.ndarray:
    """Rows whose k largest keys are distinct and strictly above the (k+1)-th."""
    srt = np.sort(keys, axis=1)[:, ::-1]
    ok = srt[:, k - 1] > srt[:, k]
    for j in range(k - 1):
        ok &= srt[:, j] > srt[:, j + 1]
    return ok


@pytest.mark.parametrize("E,k", [(128, 8), (256, 8), (32, 4)])
def test_route_lowp_matches_torch_bf16_softmax_topk_renorm(E, k):
    """softmax_topk_lowp against the reference's own sequence in bf16
    (fused_moe.py:92-96, qwen3_moe/__init__.py:473-475): F.softmax on bf16
    logits -> torch.topk -> bf16 renorm, on rows without ties in the bf16
    probabilities (torch's tie order is unspecified).  Ids must be equal and
    the weights equal bit for bit."""
    g = torch.Generator().manual_seed(E + k)
    logits = (torch.randn(512, E, generator=g) * 2.0).to(torch.bfloat16)
    p = torch.nn.functional.softmax(logits, dim=-1)
    assert p.dtype == torch.bfloat16
    tw, ti = torch.topk(p, k, dim=-1)
    tw = tw / tw.sum(dim=-1, keepdim=True)
    ids, w = O.route(logits.float().numpy(), k, "softmax_topk_lowp", True, weight_dt="bf16", prob_dt="bf16")
    ok = _tie_free_rows(p.float().numpy(), k)
    assert ok.sum() > 100
    np.testing.assert_array_equal(ids[ok], ti.numpy()[ok])
    np.testing.assert_array_equal(w[ok], tw.float().numpy()[ok])
    # the comparison separates the plausible mistakes: fp32 probabilities (the
    # softmax_topk mode) and a renorm whose sum is not rounded to bf16
    _, w32 = O.route(logits.float().numpy(), k, "softmax_topk", True)
    assert not np.array_equal(w32[ok], tw.float().numpy()[ok])
    top = torch.topk(p, k, dim=-1)[0].float()
    w_sum32 = (top / top.sum(dim=-1, keepdim=True)).to(torch.bfloat16).float().numpy()
    assert not np.array_equal(w_sum32[ok], tw.float().numpy()[ok])


# ------------------------------------------------------------------ activations
_GRID = np.concatenate([np.linspace(-12.0, 12.0, 481), [-80.0, -30.0, -1e-6, 0.0, 1e-6, 30.0, 80.0]])


@pytest.mark.parametrize("name,fn", [("silu", torch.nn.functional.silu), ("gelu", torch.nn.functional.gelu),
                                     ("relu", torch.nn.functional.relu)])
def test_activation_matches_torch(name, fn):
    """The oracle's gate activations against torch's (fused_moe.py:53-61 calls
    F.silu / F.gelu (erf form) / F.relu), float64, times a varying up value."""
    u = np.linspace(-3.0, 3.0, _GRID.size)
    got = O.act(name, _GRID, u)
    want = (fn(torch.from_numpy(_GRID)) * torch.from_numpy(u)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-300)


def test_clamped_glu_reduces_to_silu_without_limit():
    """gpt-oss's clamped GLU (gpt_oss/__init__.py:306-310) with no clamp is
    (u + 1) * g * sigmoid(alpha g) = (u + 1) * silu(alpha g) / alpha."""
    u = np.linspace(-4.0, 4.0, _GRID.size)
    for alpha in (1.0, 1.702):
        got = O.act("swiglu_oai", _GRID, u, alpha=alpha, limit=np.inf)
        silu = torch.nn.functional.silu(torch.from_numpy(_GRID * alpha)).numpy() / alpha
        np.testing.assert_allclose(got, (u + 1.0) * silu, rtol=1e-12, atol=1e-300)


def test_clamped_glu_at_and_beyond_the_limit():
    """gate clamped from above only, up from both sides: past +-limit the value
    equals the value at the limit; below -limit the gate is not clamped."""
    L, a = 7.0, 1.702
    at = O.act("swiglu_oai", [L], [L], alpha=a, limit=L)[0]
    for g, u in ((7.5, 7.0), (7.0, 9.0), (1e6, 1e6)):
        assert O.act("swiglu_oai", [g], [u], alpha=a, limit=L)[0] == at
    lo = O.act("swiglu_oai", [1.5], [-L], alpha=a, limit=L)[0]
    assert O.act("swiglu_oai", [1.5], [-20.0], alpha=a, limit=L)[0] == lo  # u clamped to -7: (u + 1) = -6
    assert lo == pytest.approx(-6.0 * torch.nn.functional.silu(torch.tensor(1.5 * a, dtype=torch.float64)).item() / a,
                               rel=1e-12)
    # the gate has no lower clamp: g = -20 keeps its (tiny, negative) value
    g = -20.0
    want = (0.5 + 1.0) * torch.nn.functional.silu(torch.tensor(g * a, dtype=torch.float64)).item() / a
    assert O.act("swiglu_oai", [g], [0.5], alpha=a, limit=L)[0] == pytest.approx(want, rel=1e-12)


# ------------------------------------------------------------------ layer
def _brute_layer(spec, x_bits, ids, w):
    """Independent float64 restatement: dense numpy dequant + per-token loops."""
    from ftmoe import synthetic  # noqa: F401  (only for the config shapes)

    x = O.bf16_bits_to_f32(x_bits).astype(np.float64)
    T, H = x.shape
    I = spec["I"]
    out = np.zeros((T, H))

    def dense(P, slot):
        if P.fmt == "fp8_block":
            return O.dequantize_block_fp8(P.w[slot], P.s[slot], P.group)
        if P.fmt == "gptq_int4":
            return O.dequantize_gptq_int4(P.w[slot], P.z[slot], P.s[slot], P.group).T
        if P.fmt == "int8_channel":
            return O.dequantize_int8_packed(P.w[slot], P.s[slot], P.K)
        if P.fmt == "mxfp4":
            return O.dequantize_mxfp4_blocks(P.w[slot], P.s[slot])
        return O.bf16_bits_to_f32(P.w[slot])

    def bias(P, slot):
        return 0.0 if P.bias is None else O.bf16_bits_to_f32(P.bias[slot]).astype(np.float64)

    for t in range(T):
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            W13 = dense(spec["w13"], e).astype(np.float64)
            W2 = dense(spec["w2"], e).astype(np.float64)
            gu = W13 @ x[t] + bias(spec["w13"], e)
            g, u = gu[:I], gu[I:]
            if spec["act"] == "swiglu_oai":
                g = np.minimum(g, spec["limit"])
                u = np.clip(u, -spec["limit"], spec["limit"])
                h = (u + 1) * g / (1 + np.exp(-spec["alpha"] * g))
            else:
                h = g / (1 + np.exp(-g)) * u
            h = O.round_bf16(h.astype(np.float32)).astype(np.float64)
            out[t] += float(w[t, j]) * (W2 @ h + bias(spec["w2"], e))
    return out


@pytest.mark.parametrize("name", ["c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"])
def test_layer_oracle_matches_float64_brute_force(name):
    from ftmoe import synthetic as S

    cfg = S.SMALL[name]
    syn = S.generate(cfg, T=3, seed=7)
    spec = oracle_spec(syn)
    spec.pop("shared", None)
    res = O.layer_reference(spec, np_(syn.x))
    brute = _brute_layer(spec, np_(syn.x), res["ids"], res["w"])
    # both in float64; h is rounded to bf16 in both, so only summation order differs
    np.testing.assert_allclose(res["out"], brute, rtol=1e-6, atol=1e-9)


@pytest.mark.skipif(not O.ref_cpu_moe_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_experts_match_reference_cpu_moe_kernel():
    """SwiGLU + weighted combine against freetoken_cpu_moe_forward_fast
    (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:470-528,763-786) on the
    oracle's fp32 dequantized banks (h kept fp32 there, as cpu_moe.cpp does)."""
    from ftmoe import synthetic as S

    cfg = S.SMALL["c3_fp8"]
    syn = S.generate(cfg, T=6, seed=3)
    spec = oracle_spec(syn)
    x = O.bf16_bits_to_f32(np_(syn.x))
    logits = O.router_logits(np_(syn.x), spec["gate_w"])
    ids, w = O.route(logits, cfg.k)
    gu = np.stack([O.dequant(spec["w13"], e) for e in range(cfg.E)])
    dn = np.stack([O.dequant(spec["w2"], e) for e in range(cfg.E)])
    ref = O.ref_cpu_moe_forward_fast(x, ids, w, gu, dn, threads=1)
    got = O.moe_experts(spec["w13"], spec["w2"], x, ids, w, E=cfg.E, h_bf16=False)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ routing arithmetic (replayed from the GPU)
# The oracle's routing runs the kernel's IEEE operations step for step
# (orc_route: its own e^x, the per-lane and DPP-tree sums), so GPU routing
# indices and weights are compared bit for bit.  These tests pin that
# restatement against the mathematics it must compute.
_LOG2E, _LN2_HI, _LN2_LO = 1.4426950216293335, 0.6931471824645996, 1.9046542121259336e-09


def _ulp32(t):
    """ulp of fp32 at the (normal, non-zero) float64 values t."""
    e = np.floor(np.log2(np.abs(t)))
    return np.ldexp(1.0, (e - 23).astype(np.int64))


def _exp_inputs():
    rng = np.random.RandomState(0)
    k = np.arange(-150, 129)
    return np.concatenate([
        rng.uniform(-104.0, 88.7, 400_000), rng.uniform(-1.0, 1.0, 100_000), rng.uniform(-1e-3, 1e-3, 20_000),
        k * np.log(2.0), k * np.log(2.0) + 1e-6, k * np.log(2.0) - 1e-6, (k + 0.5) * np.log(2.0),
        [0.0, -0.0, -87.33654, -87.3, -103.9, -100.0, 88.72, 1e-30, -1e-30],
    ]).astype(np.float32)


def _emulated_exp(x, *, drop_lo=False, lo_sign=1.0, degree=7, half=0.5):
    """The routing e^x restated in numpy (each fused multiply-add taken in
    float64 and rounded once to fp32), with a switch per plausible slip."""
    from math import factorial

    f32 = np.float32
    x = np.clip(np.asarray(x, f32), f32(-104.0), f32(89.0))
    fma = lambda a, b, c: (a.astype(np.float64) * np.float64(b) + c.astype(np.float64)).astype(f32)
    n = np.rint(x * f32(_LOG2E)).astype(f32)
    r = fma(n, -f32(_LN2_HI), x)
    if not drop_lo:
        r = fma(n, f32(lo_sign * _LN2_LO), r)
    coefs = [f32(1.0 / factorial(j)) for j in range(degree, 1, -1)]
    coefs[-1] = f32(half)
    p = np.full_like(r, coefs[0])
    for c in coefs[1:]:
        p = fma(p, r, np.full_like(r, c))
    p = fma(p, r, np.ones_like(r))
    p = fma(p, r, np.ones_like(r))
    with np.errstate(over="ignore"):
        return np.ldexp(p.astype(np.float64), n.astype(np.int64)).astype(f32)


def _max_ulp_err(got, x):
    ref = np.exp(np.asarray(x, np.float64))
    normal = (ref >= 2.0 ** -126) & (ref <= np.finfo(np.float32).max)
    return float(np.max(np.abs(got[normal].astype(np.float64) - ref[normal]) / _ulp32(ref[normal]))), ref, normal


def test_routing_exp_is_faithful_against_float64():
    """orc_expf (Cody-Waite reduction, degree-7 Taylor in Horner form) is
    within one ulp of e^x wherever the result is normal, within one
    subnormal quantum below that, exact at 0, 0 past the underflow point and
    inf past FLT_MAX."""
    x = _exp_inputs()
    got = O.expf(x)
    err, ref, normal = _max_ulp_err(got, x)
    assert err <= 1.0, err
    sub = ref < 2.0 ** -126
    assert np.all(np.abs(got[sub].astype(np.float64) - ref[sub]) <= 2.0 ** -149)
    assert np.isinf(got[ref > np.finfo(np.float32).max]).all()
    assert O.expf(np.float32([0.0, -0.0]))[0] == 1.0 == O.expf(np.float32([-0.0]))[0]
    assert O.expf(np.float32([-104.0, -200.0, -np.inf]))[0] == 0.0
    assert np.all(O.expf(np.float32([-104.0, -200.0, -np.inf])) == 0.0)
    assert np.isinf(O.expf(np.float32([89.0, 1e4]))).all()


@pytest.mark.parametrize("slip", ["none", "drop_lo", "lo_sign", "degree5", "half"])
def test_routing_exp_check_catches_plausible_slips(slip):
    """The one-ulp bound above separates the routine from the slips a
    restatement could make: the low part of ln 2 dropped or of the wrong sign,
    two Taylor terms lost, a wrong coefficient."""
    x = _exp_inputs()
    kw = {"none": {}, "drop_lo": {"drop_lo": True}, "lo_sign": {"lo_sign": -1.0}, "degree5": {"degree": 5},
          "half": {"half": 0.5 + 2.0 ** -10}}[slip]
    err = _max_ulp_err(_emulated_exp(x, **kw), x)[0]
    if slip == "none":
        assert err <= 1.0, err
    else:
        assert err > 1.0, (slip, err)


def test_wave_sum_takes_every_lane_once():
    """The DPP-tree order adds each of the 64 lanes exactly once: a one-hot
    vector returns its value, integer vectors (every partial sum exact) return
    the exact total, and random vectors stay within the fp32 bound of the
    float64 sum."""
    for lane in range(64):
        v = np.zeros(64, np.float32)
        v[lane] = 3.0
        assert O.wave_sum(v) == 3.0, lane
    v = np.arange(1, 65, dtype=np.float32) * np.float32(7.0)
    assert O.wave_sum(v) == 7.0 * 64 * 65 / 2
    rng = np.random.RandomState(1)
    for _ in range(50):
        v = rng.rand(64).astype(np.float32) * np.float32(rng.choice([1e-3, 1.0, 1e3]))
        exact = float(np.sum(v.astype(np.float64)))
        assert abs(O.wave_sum(v) - exact) <= 6 * 2.0 ** -24 * exact


def test_f16_rounding_matches_numpy():
    """orc_round_f16 (the LOWP probabilities in fp16 logits' dtype) is
    numpy's round-to-nearest-even binary16 conversion, subnormals and overflow
    included."""
    rng = np.random.RandomState(2)
    edge = np.float32([65504.0, 65519.99, 65520.0, 7e4, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14,
                       2.0 ** -14 - 2.0 ** -25, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 0.0, -0.0, -1.5e-6])
    x = np.concatenate([edge, -edge, (rng.randn(20000) * np.float32(10.0) ** rng.randint(-8, 5, 20000))
                        .astype(np.float32)])
    got = np.array([O.lib().orc_round_f16(float(v)) for v in x], np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _boundary_free_rows(keys, k, margin):
    """Rows whose k-th key exceeds the (k+1)-th by more than ``margin`` (relative)
    and whose top k are distinct by the same margin."""
    srt = np.sort(keys, axis=1)[:, ::-1].astype(np.float64)
    ok = srt[:, k - 1] > srt[:, k] * (1 + margin) + 1e-30
    for j in range(k - 1):
        ok &= srt[:, j] > srt[:, j + 1] * (1 + margin) + 1e-30
    return ok


@pytest.mark.parametrize("mode", ["softmax_topk", "softmax_topk_lowp", "topk_softmax"])
@pytest.mark.parametrize("E,k", [(16, 2), (32, 4), (100, 6), (128, 8), (256, 8)])
def test_route_replay_agrees_with_float64_routing(mode, E, k):
    """orc_route against the textbook float64 softmax / top-k / renorm
    (route_f64): the same experts wherever no key sits within rounding
    distance of the top-k boundary; fp32 weights within 4 ulp, and in LOWP
    mode (every rounding in bf16) within one bf16 ulp."""
    g = torch.Generator().manual_seed(E * 10 + k)
    logits = (torch.randn(400, E, generator=g) * 2.0).to(torch.bfloat16).float().numpy()
    wdt = "bf16" if mode == "softmax_topk_lowp" else "f32"
    ids, w = O.route(logits, k, mode, True, weight_dt=wdt)
    ids64, w64 = O.route_f64(logits, k, mode, True, weight_dt=wdt)
    if mode == "softmax_topk_lowp":
        m = logits.max(axis=1, keepdims=True)
        e = np.exp((logits - m).astype(np.float64))
        keys = e / e.sum(axis=1, keepdims=True)
        ok = _boundary_free_rows(keys, k, 2.0 ** -6)
    else:
        ok = _boundary_free_rows(logits - logits.min(axis=1, keepdims=True) + 1.0, k, 1e-9)
    assert ok.sum() > 50
    np.testing.assert_array_equal(ids[ok], ids64[ok])
    tol = 2.0 ** -7 if mode == "softmax_topk_lowp" else 4 * 2.0 ** -23
    np.testing.assert_allclose(w[ok], w64[ok], rtol=tol, atol=0)


def test_route_renorm_off_and_f16_probabilities():
    """renormalize=False returns the probabilities themselves; fp16 logits
    take their LOWP probabilities in fp16."""
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(64, 40, generator=g).to(torch.float16).float().numpy()
    ids, w = O.route(logits, 4, "softmax_topk_lowp", False, weight_dt="f32", prob_dt="f16")
    m = logits.max(axis=1, keepdims=True)
    e = np.exp((logits - m).astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32).astype(np.float16).astype(np.float32)
    ok = _boundary_free_rows(p, 4, 2.0 ** -9)
    np.testing.assert_allclose(w[ok], np.take_along_axis(p, ids, 1)[ok], rtol=2.0 ** -10, atol=0)
    ids, w = O.route(logits, 4, "softmax_topk", False, weight_dt="f32")
    np.testing.assert_allclose(w, np.take_along_axis(e / e.sum(1, keepdims=True), ids, 1), rtol=4 * 2.0 ** -23)


# ------------------------------------------------------------------ shared expert and on_input, brute force
def _shared_brute(x_bits, sh):
    """sigmoid(x . g_s) * down(silu(gate x) * up x) in float64
    (qwen3_5_moe/__init__.py:1229-1230, 1766-1768), from the bf16 weights:
    the gate logit and the weight rounded to bf16 (bf16 Linear, bf16
    sigmoid), h rounded to bf16."""
    x = O.bf16_bits_to_f32(x_bits).astype(np.float64)
    W13 = O.bf16_bits_to_f32(sh["w13"]).astype(np.float64)
    W2 = O.bf16_bits_to_f32(sh["w2"]).astype(np.float64)
    gs = O.bf16_bits_to_f32(sh["gate"]).astype(np.float64)
    Is = W2.shape[1]
    logit = O.round_bf16((x @ gs.T).astype(np.float32)).astype(np.float64)[:, 0]
    sw = O.round_bf16((1.0 / (1.0 + np.exp(-logit))).astype(np.float32)).astype(np.float64)
    gu = x @ W13.T
    g, u = gu[:, :Is], gu[:, Is:]
    h = O.round_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32)).astype(np.float64)
    return sw, h @ W2.T


def test_shared_expert_branch_matches_float64_brute_force():
    """layer_reference's shared-expert branch against an independent float64
    restatement: the gate weight bit for bit, the layer within summation-order
    rounding.  A missing sigmoid, a missing gate, or the gate applied to the
    routed sum instead fail the same comparison."""
    from ftmoe import synthetic as S

    syn = S.generate(S.SMALL["c3_fp8"], T=5, seed=21)
    assert syn.shared is not None
    spec = oracle_spec(syn)
    xb = np_(syn.x)
    res = O.layer_reference(spec, xb)
    sw, ys = _shared_brute(xb, spec["shared"])
    np.testing.assert_array_equal(res["shared_w"], sw.astype(np.float32))
    routed = _brute_layer({k: v for k, v in spec.items() if k != "shared"}, xb, res["ids"], res["w"])
    brute = routed + sw[:, None] * ys
    np.testing.assert_allclose(res["out"], brute, rtol=1e-6, atol=1e-9)
    logit = O.router_logits(xb, spec["shared"]["gate"])[:, 0].astype(np.float64)
    slips = {"no sigmoid": routed + logit[:, None] * ys, "no gate": routed + ys,
             "gate on the sum": sw[:, None] * (routed + ys)}
    for name, wrong in slips.items():
        assert not np.allclose(res["out"], wrong, rtol=1e-3, atol=1e-6), name


def test_router_weight_on_input_matches_float64_brute_force():
    """apply_router_weight_on_input (fused_moe.py:139-148): the expert runs on
    round_bf16(w * x) and its output is not weighted again.  Checked against a
    float64 per-pair restatement; the weight applied after w2 (the default
    path) or applied twice fails the comparison."""
    rng = np.random.RandomState(4)
    E, H, I, T, k = 6, 64, 32, 5, 2
    w1 = O.f32_to_bf16_bits((rng.randn(E, 2 * I, H) * 0.1).astype(np.float32))
    w2 = O.f32_to_bf16_bits((rng.randn(E, H, I) * 0.1).astype(np.float32))
    xb = O.f32_to_bf16_bits(rng.randn(T, H).astype(np.float32))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = O.round_bf16(rng.uniform(0.1, 0.9, (T, k)).astype(np.float32))
    p13, p2 = O.OracleProj("bf16", w1, 2 * I, H), O.OracleProj("bf16", w2, H, I)
    x = O.bf16_bits_to_f32(xb)
    got = O.moe_experts(p13, p2, x, ids, w, E=E, on_input=True)

    def brute(on_input, after):
        out = np.zeros((T, H))
        for t in range(T):
            for j in range(k):
                e = ids[t, j]
                xi = O.round_bf16((x[t] * w[t, j]).astype(np.float32)) if on_input else x[t]
                gu = O.bf16_bits_to_f32(w1[e]).astype(np.float64) @ xi.astype(np.float64)
                g, u = gu[:I], gu[I:]
                h = O.round_bf16((g / (1 + np.exp(-g)) * u).astype(np.float32)).astype(np.float64)
                y = O.bf16_bits_to_f32(w2[e]).astype(np.float64) @ h
                out[t] += (float(w[t, j]) if after else 1.0) * y
        return out

    np.testing.assert_allclose(got, brute(True, False), rtol=1e-6, atol=1e-9)
    for name, wrong in {"weight after w2": brute(False, True), "weight twice": brute(True, True)}.items():
        assert not np.allclose(got, wrong, rtol=1e-2, atol=1e-4), name


@pytest.mark.parametrize("E,k", [(128, 8), (256, 8)])
def test_lowp_adversarial_rows_are_arithmetic_sensitive(E, k):
    """The adversarial LOWP batch the GPU routing tests use: most rows put a
    boundary probability within one fp32 ulp of a bf16 midpoint, many tie
    across the boundary, and on a good share the textbook float64 routing
    selects other experts than the replayed fp32 arithmetic -- so only
    bit-identical arithmetic can reproduce the oracle's ids on them."""
    from lowp_adversarial import adversarial_logits, boundary_stats

    L = adversarial_logits(512, E, k, seed=E)
    st = boundary_stats(L, k)
    assert st["near_midpoint"] >= 200, st
    assert st["boundary_ties"] >= 100, st
    ids, _ = O.route(L, k, "softmax_topk_lowp", True)
    ids64, _ = O.route_f64(L, k, "softmax_topk_lowp", True)
    assert (ids != ids64).any(1).sum() >= 20
