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
