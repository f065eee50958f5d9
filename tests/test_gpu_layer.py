"""GPU: the whole fused MoE layer through the C ABI against the oracle.

Routing indices, router logits and router weights are bit-exact (the
oracle replays the router kernel's fp32 summation order, its e^x routine and
its softmax sums operation for operation); the bf16 layer output is within
|got - ref| <= 2e-2 + 1e-2 |ref| of the fp32-accumulated oracle.  Covers all
four quantized formats at reduced shapes, the FP8 + shared-expert layer (C3)
and the INT8 layer (C1) at their full shapes, caller-supplied routing, the
dense ``fused`` backend, and run-to-run bitwise determinism."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import ATOL, MX_REL_RMS, RTOL, assert_close, np_, oracle_spec, rel_rms, to_f32, wide_range_x

from ftmoe import _native as nat
from ftmoe import synthetic as S

pytestmark = pytest.mark.gpu


def _run_and_check(syn, gpu, *, check_routing=True):
    spec = oracle_spec(syn)
    ref = O.layer_reference(spec, np_(syn.x))
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    out, ids, w, logits = layer.forward(dsyn.x, return_routing=True)
    torch.cuda.synchronize()
    if check_routing:
        np.testing.assert_array_equal(to_f32(logits), ref["logits"], err_msg="router logits")
        np.testing.assert_array_equal(ids.cpu().numpy(), ref["ids"], err_msg="routing indices")
        np.testing.assert_array_equal(w.cpu().numpy(), ref["w"], err_msg="router weights")
    assert_close(to_f32(out), ref["out"], what=f"{syn.cfg.name} layer output")
    return layer, dsyn, ref, out


@pytest.mark.parametrize("name", ["c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"])
@pytest.mark.parametrize("T", [1, 5, 16, 21, 24])
def test_small_layer_matches_oracle(gpu, name, T):
    syn = S.generate(S.SMALL[name], T=T, seed=11 + T)
    _run_and_check(syn, gpu)


@pytest.mark.parametrize("Is,T", [(128, 1), (128, 6), (128, 16), (128, 20), (128, 40), (1408, 1), (1408, 9),
                                  (1408, 20)])
def test_gptq_layer_with_shared_expert_matches_oracle(gpu, Is, T):
    """GPTQ routed experts beside a dense shared expert: the GPTQ decode
    stages (stage A up to 16 tokens, stage B up to 32) run the shared
    expert's items on their bf16 path (stage B: 16 columns, K split over 4
    waves, tokens in blocks of 8; at 1408 a wave's K quarter takes several
    prefetch windows), the register-fed ones above."""
    from dataclasses import replace

    syn = S.generate(replace(S.SMALL["c2_gptq"], shared_inter=Is), T=T, seed=40 + T + Is)
    _run_and_check(syn, gpu)


@pytest.mark.parametrize("name,T", [("c2_gptq", 9), ("c3_fp8", 9), ("c4_mxfp4", 9), ("c3_fp8", 80)])
def test_small_layer_routed_matches_oracle(gpu, name, T):
    """Caller-supplied routing; at T=80 the shared-gate logit comes from the
    row-blocked router over the single shared row."""
    syn = S.generate(S.SMALL[name], T=T, seed=5)
    spec = oracle_spec(syn)
    rng = np.random.RandomState(0)
    ids = np.stack([rng.choice(syn.cfg.E, syn.cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
    w = O.round_bf16(rng.rand(T, syn.cfg.k).astype(np.float32))
    ref = O.layer_reference(spec, np_(syn.x), ids=ids, w=w)
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    out = layer.forward_routed(dsyn.x, torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu))
    assert_close(to_f32(out), ref["out"], what="routed layer")


def test_layer_is_bitwise_deterministic(gpu):
    syn = S.generate(S.SMALL["c3_fp8"], T=16, seed=3).to(gpu)
    layer = S.build_layer(syn)
    a = layer.forward(syn.x)
    b = layer.forward(syn.x)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.fixture(scope="module")
def c3_full():
    return S.generate(S.CONFIGS["c3_fp8"], T=64, seed=0)


@pytest.mark.parametrize("T", [1, 4, 16, 37, 64])
def test_c3_fp8_full_shape_matches_oracle(gpu, c3_full, T):
    base = c3_full
    syn = S.SyntheticLayer(base.cfg, base.bank, base.gate_w, base.x[:T].contiguous(), shared=base.shared)
    _run_and_check(syn, gpu)


@pytest.fixture(scope="module")
def c2_full():
    return S.generate(S.CONFIGS["c2_gptq"], T=64, seed=1)


@pytest.mark.parametrize("T", [1, 4, 16, 32, 64])
def test_c2_gptq_full_shape_matches_oracle(gpu, c2_full, T):
    """GPTQ int4 g128 at the C2 shape (128 experts, top-8): the decode stages
    with rows in LDS (stage A: 8 groups per wave up to 16 tokens; stage B: 3
    groups per wave up to 32) and the register-fed stages at 64."""
    base = c2_full
    syn = S.SyntheticLayer(base.cfg, base.bank, base.gate_w, base.x[:T].contiguous(), shared=base.shared)
    _run_and_check(syn, gpu)


@pytest.fixture(scope="module")
def c4_full(gpu):
    # drawn and quantized on the GPU (423 MB of MXFP4 banks: about a minute on the host)
    return S.generate(S.CONFIGS["c4_mxfp4"], T=128, seed=2, device=gpu)


@pytest.mark.parametrize("T", [1, 16, 32, 128])
def test_c4_mxfp4_full_shape_matches_oracle(gpu, c4_full, T):
    """MXFP4 at the C4 shape (H = I = 2880, 32 experts, top-4 on biased logits,
    clamped SwiGLU with biases): stage A on scaled MFMAs with activations in
    LDS (16-channel items at T = 1, 8-channel above) and stage B with K split
    over the waves up to 16 tokens per expert (T = 128)."""
    from dataclasses import replace

    _run_and_check(replace(c4_full, x=c4_full.x[:T].contiguous()), gpu)


@pytest.mark.parametrize("T", [1, 4, 13, 32])
def test_mxfp4_decode_wide_range_inputs(gpu, T):
    """The MXFP4 decode stage A feeds the input to scaled fp8 x fp4 MFMAs as
    two e4m3 terms per element: with elements spanning 2^-14 .. 2^3 inside
    every 32-wide block the output stays at bf16 precision (relative RMS
    error MX_REL_RMS; one e4m3 term would give about 3e-2).  H = 320 is not a
    multiple of the 128-wide chunks (zero-padded tail)."""
    from dataclasses import replace

    syn = S.generate(S.SMALL["c4_mxfp4"], T=T, seed=50 + T)
    syn = replace(syn, x=wide_range_x(T, syn.cfg.H, seed=T))
    _, _, ref, out = _run_and_check(syn, gpu)
    err = rel_rms(to_f32(out), ref["out"])
    assert err < MX_REL_RMS, err


@pytest.mark.parametrize("T", [64, 200, 256])
def test_mxfp4_many_experts_lds_path(gpu, T):
    """MXFP4 on 128 experts, top-2 (1 to 4 tokens per expert): the scaled-MFMA
    stage A and the K-split stage B up to 256 tokens, the input quantised by
    the router-rows launch, the work records written by the multi-workgroup
    top-k (64, 200) and the block top-k (256)."""
    from dataclasses import replace

    syn = S.generate(replace(S.SMALL["c4_mxfp4"], E=128, k=2), T=T, seed=60 + T)
    _run_and_check(syn, gpu)


@pytest.mark.parametrize("T,hot", [(16, False), (48, False), (64, False), (64, True)])
def test_mxfp4_token_resident_stages(gpu, T, hot):
    """MXFP4 at 4 to 16 tokens per routed expert: both projections on
    k_stage_tok_a / _b (one block of up to 32 token rows of an expert in LDS per
    workgroup, 8 waves of 16 weight rows each over the whole K, 320 and 192
    not multiples of the 128-wide wave-loads).  hot: a gate bias of 8 on
    expert 0 routes every token to it, so its 64 tokens take two blocks and
    its weights are streamed twice."""
    from dataclasses import replace

    syn = S.generate(S.SMALL["c4_mxfp4"], T=T, seed=80 + T)
    if hot:
        gb = syn.gate_b.clone()
        gb[0] = 8.0
        syn = replace(syn, gate_b=gb)
    layer, _, ref, _ = _run_and_check(syn, gpu)
    assert layer.stage_kernel(T, nat.STAGE_W13) == "k_stage_tok_a"
    assert layer.stage_kernel(T, nat.STAGE_W2) == "k_stage_tok_b"
    if hot:
        assert (ref["ids"] == 0).any(axis=1).all()


def test_c4_mxfp4_full_shape_wide_range_inputs(gpu, c4_full):
    from dataclasses import replace

    syn = replace(c4_full, x=wide_range_x(32, c4_full.cfg.H, seed=99).to(gpu))
    _, _, ref, out = _run_and_check(syn, gpu)
    err = rel_rms(to_f32(out), ref["out"])
    assert err < MX_REL_RMS, err


def test_c4_mxfp4_prefill_token_subset(gpu, c4_full):
    """C4 at its prefill size (T=4096 through the MXFP4 GEMM tiles): a token's
    output depends only on its own row, so 40 sampled tokens are checked
    against the oracle run on just those rows; routing bit-exact."""
    from dataclasses import replace

    g = torch.Generator(device=gpu).manual_seed(4096)
    x = torch.randn(4096, c4_full.cfg.H, generator=g, device=gpu).to(torch.bfloat16)
    syn = replace(c4_full, x=x)
    layer = S.build_layer(syn)
    out, ids, _, _ = layer.forward(x, return_routing=True)
    torch.cuda.synchronize()
    rows = np.sort(np.random.RandomState(1).choice(4096, 40, replace=False))
    ref = O.layer_reference(oracle_spec(syn), np_(x)[rows])
    np.testing.assert_array_equal(ids.cpu().numpy()[rows], ref["ids"])
    assert_close(to_f32(out)[rows], ref["out"], what="C4 prefill rows")


def test_c1_int8_full_shape_matches_oracle(gpu):
    syn = S.generate(S.CONFIGS["c1_int8"], T=4, seed=0)
    _run_and_check(syn, gpu)


def test_expert_forward_single_slot(gpu):
    syn = S.generate(S.SMALL["c3_fp8"], T=7, seed=9)
    spec = oracle_spec(syn)
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    for slot in (0, 5, syn.cfg.E - 1):
        got = layer.expert_forward(slot, dsyn.x)
        ref = O.expert_forward(spec["w13"], spec["w2"], slot, O.bf16_bits_to_f32(np_(syn.x)))
        assert_close(to_f32(got), ref, what=f"expert {slot}")


# ---------------------------------------------------------------- fused backend (dense banks)
def _fused_ref(x, w1, w2, gating, k, renorm, act, on_input, wdt):
    """Oracle for fused_moe.py:64-161 on dense banks."""
    E, I2, H = w1.shape
    xb = x.float().numpy()
    ids, w = O.route(gating.float().numpy(), k, "softmax_topk_lowp", renorm,
                     weight_dt="bf16" if x.dtype == torch.bfloat16 else "f32",
                     prob_dt="bf16" if gating.dtype == torch.bfloat16 else "f32")
    fmt = "bf16" if wdt == torch.bfloat16 else "fp32"
    a = np_(w1) if fmt == "bf16" else w1.float().numpy()
    b = np_(w2) if fmt == "bf16" else w2.float().numpy()
    p13 = O.OracleProj(fmt, np.ascontiguousarray(a), I2, H)
    p2 = O.OracleProj(fmt, np.ascontiguousarray(b), H, I2 // 2)
    bf = x.dtype == torch.bfloat16
    return O.moe_experts(p13, p2, xb, ids, w, E=E, act=act, h_bf16=bf, on_input=on_input, x_bf16=bf)


@pytest.mark.parametrize("renorm,act,on_input", [(True, "silu", False), (True, "silu", True), (False, "gelu", False)])
def test_fused_backend_fp32_tiny(gpu, renorm, act, on_input):
    """tests/test_moe_fused.py:58-181 shapes (E=5, H=7, I=4, T=6, k=2) at atol 1e-5."""
    from ftmoe.moe import create_moe_backend

    g = torch.Generator().manual_seed(1)
    E, H, I, T, K = 5, 7, 4, 6, 2
    w1, w2 = torch.randn(E, 2 * I, H, generator=g), torch.randn(E, H, I, generator=g)
    x, gating = torch.randn(T, H, generator=g), torch.randn(T, E, generator=g)
    backend = create_moe_backend("fused")
    got = backend.forward(x.to(gpu), w1.to(gpu), w2.to(gpu), gating.to(gpu), K, renorm, act, on_input)
    ref = _fused_ref(x, w1, w2, gating, K, renorm, act, on_input, torch.float32)
    np.testing.assert_allclose(got.cpu().numpy(), ref, atol=1e-5, rtol=1e-5)


def test_fused_backend_bf16_serving_shape(gpu):
    from ftmoe.moe import create_moe_backend

    g = torch.Generator().manual_seed(2)
    E, H, I, T, K = 64, 1024, 256, 12, 4
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gating = torch.randn(T, E, generator=g).to(torch.bfloat16)
    got = create_moe_backend("fused").forward(x.to(gpu), w1.to(gpu), w2.to(gpu), gating.to(gpu), K, True, "silu", False)
    ref = _fused_ref(x, w1, w2, gating, K, True, "silu", False, torch.bfloat16)
    assert_close(got.float().cpu().numpy(), ref, ATOL, RTOL, what="fused bf16")


@pytest.mark.parametrize("full,T", [(False, 16), (True, 2)])
def test_stages_in_order_equal_forward(gpu, full, T):
    """ftm_moe_forward_stage 0..4 launched in order is the same computation as
    ftm_moe_forward (bitwise).  Full C3 at T=2 routes inside stage A (the
    top-k stage launches nothing)."""
    from ftmoe import _native as nat

    syn = S.generate(S.CONFIGS["c3_fp8"] if full else S.SMALL["c3_fp8"], T=T, seed=21).to(gpu)
    layer = S.build_layer(syn)
    ref = layer.forward(syn.x)
    out = torch.empty_like(syn.x)
    for st in (nat.STAGE_ROUTER, nat.STAGE_TOPK, nat.STAGE_W13, nat.STAGE_W2, nat.STAGE_COMBINE):
        layer.forward_stage(syn.x, out, st)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_graph_replay_matches_eager(gpu):
    """A layer forward captured in a HIP graph replays to the eager result, with
    eager forwards of other batches on the same layer between the replays."""
    syn = S.generate(S.SMALL["c3_fp8"], T=8, seed=22).to(gpu)
    layer = S.build_layer(syn)
    other = torch.randn(8, syn.cfg.H, device=gpu).to(torch.bfloat16)
    ref = layer.forward(syn.x)
    s = torch.cuda.Stream(device=gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        layer.forward(syn.x)  # this stream's workspace is allocated outside capture
    torch.cuda.current_stream(gpu).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = layer.forward(syn.x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        layer.forward(other)
        torch.cuda.synchronize()


def test_large_batch_multi_workgroup_topk(gpu):
    """T above the single-workgroup top-k limit takes the multi-workgroup path
    (last-arriving workgroup compacts): routing stays bit-exact."""
    syn = S.generate(S.SMALL["c3_fp8"], T=300, seed=23)
    _run_and_check(syn, gpu)


@pytest.mark.parametrize("E,k", [(320, 6), (512, 8)])
def test_many_experts_routing(gpu, E, k):
    """More than 256 experts: 8 selection candidates per lane."""
    from dataclasses import replace

    cfg = replace(S.SMALL["c3_fp8"], name=f"c3_e{E}", E=E, k=k)
    syn = S.generate(cfg, T=12, seed=24)
    _run_and_check(syn, gpu)


# ---------------------------------------------------------------- above the token crossover (tiled GEMMs)
@pytest.mark.parametrize("name,T", [("c3_fp8", 512), ("c1_int8", 256), ("c4_mxfp4", 256), ("c3_fp8", 700)])
def test_prefill_gemm_path_matches_oracle(gpu, name, T):
    """At >= 16 tokens per routed expert the expert stages are the LDS-tiled
    GEMMs (FP8 block, INT8 per-channel, MXFP4 with biases and the clamped
    SwiGLU, the bf16 shared expert); same contract as the GEMV path."""
    syn = S.generate(S.SMALL[name], T=T, seed=40 + T)
    _run_and_check(syn, gpu)


@pytest.mark.parametrize("H,I,bias", [(384, 384, False), (256, 128, False), (256, 256, True), (640, 512, False)])
def test_fp8_prefill_register_fed_stage_b_shapes(gpu, H, I, bias):
    """FP8 above the crossover with stage B on the register-fed tile
    (k_gemm_mxb_f8, asserted by name): K = I of three, one, two and four
    128-wide steps (the tile unrolls four), an odd number of 128-column N
    tiles (H = 384, 640: 3 and 5; the workgroup's last N tile is then past
    its range), bf16 expert biases (the tile's 16-bit bias loads).  Its
    output equals the ring tile's stage B (k_gemm_mx, forced by
    FTM_PROJ_RING_B on the same banks) bit for bit."""
    from dataclasses import replace

    from ftmoe import _native as nat

    cfg = replace(S.SMALL["c3_fp8"], name=f"c3_h{H}_i{I}", H=H, I=I, expert_bias=bias)
    syn = S.generate(cfg, T=512, seed=90 + I + H)
    layer, dsyn, ref, out = _run_and_check(syn, gpu)
    assert layer.stage_kernel(512, nat.STAGE_W2) == "k_gemm_mxb_f8"
    ring = S.build_layer(dsyn)
    ring.w2.flags = nat.PROJ_RING_B
    assert ring.stage_kernel(512, nat.STAGE_W2) == "k_gemm_mx"
    out_ring = ring.forward(dsyn.x)
    torch.cuda.synchronize()
    assert torch.equal(out_ring, out)


@pytest.mark.parametrize("T", [256, 600])
def test_mxfp4_tiles_wide_range_inputs(gpu, T):
    """MXFP4 above the crossover: stage A on the scaled-MFMA tiles (128-token
    M tiles, partly filled at 64 and 150 tokens per expert; H = 320 ends in a
    half K step) with inputs spanning 2^-14 .. 2^3 inside each 32-wide block:
    the output stays at bf16 precision (relative RMS MX_REL_RMS).  Caller
    routing then quantises the input in its own launch (no router launch)."""
    from dataclasses import replace

    syn = S.generate(S.SMALL["c4_mxfp4"], T=T, seed=70 + T)
    syn = replace(syn, x=wide_range_x(T, syn.cfg.H, seed=T))
    layer, dsyn, ref, out = _run_and_check(syn, gpu)
    err = rel_rms(to_f32(out), ref["out"])
    assert err < MX_REL_RMS, err
    ids = torch.from_numpy(np.ascontiguousarray(ref["ids"], np.int32)).to(gpu)
    w = torch.from_numpy(np.ascontiguousarray(ref["w"], np.float32)).to(gpu)
    out_r = layer.forward_routed(dsyn.x, ids, w)
    torch.cuda.synchronize()
    assert_close(to_f32(out_r), ref["out"], what="MXFP4 tiles, caller routing")


def test_prefill_gemm_full_c3_token_subset(gpu):
    """C3 at its prefill size (T=2048, all 256 experts hit): the layer runs on
    the whole batch; a token's output depends only on its own row, so 48
    sampled tokens are checked against the oracle run on just those rows."""
    syn = S.generate(S.CONFIGS["c3_fp8"], T=2048, seed=7)
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    out, ids, _, _ = layer.forward(dsyn.x, return_routing=True)
    torch.cuda.synchronize()
    rows = np.sort(np.random.RandomState(0).choice(2048, 48, replace=False))
    ref = O.layer_reference(oracle_spec(syn), np_(syn.x)[rows])
    np.testing.assert_array_equal(ids.cpu().numpy()[rows], ref["ids"])
    assert_close(to_f32(out)[rows], ref["out"], what="C3 prefill rows")
    again = layer.forward(dsyn.x)
    torch.cuda.synchronize()
    assert torch.equal(out, again)


@pytest.mark.parametrize("T", [2, 9])
def test_non_resident_expert_contributes_zero_and_flags(gpu, T):
    """A routed expert whose slot is -1 (not resident in an offload pool)
    contributes nothing to its tokens and sets bit 0 of the workspace error
    word; the rest of the layer is unaffected.  T=2 takes the decode stages
    with activations in LDS, T=9 the register-fed ones."""
    from ftmoe.layer import workspace

    syn = S.generate(S.SMALL["c3_fp8"], T=T, seed=50 + T)
    spec = oracle_spec(syn)
    ref_full = O.layer_reference(spec, np_(syn.x))
    ids = ref_full["ids"].astype(np.int32)
    w = ref_full["w"].astype(np.float32)
    missing = int(ids[0, 0])
    w_ref = np.where(ids == missing, 0.0, w).astype(np.float32)
    ref = O.layer_reference(spec, np_(syn.x), ids=ids, w=w_ref)
    dsyn = syn.to(gpu)
    slots = torch.arange(syn.cfg.E, dtype=torch.int32, device=gpu)
    slots[missing] = -1
    layer = S.build_layer(dsyn, slot_of_expert=slots)
    ws = workspace(gpu, layer.workspace_bytes(T))
    ws[:16].zero_()
    out = layer.forward_routed(dsyn.x, torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu))
    torch.cuda.synchronize()
    err = int(ws[12:16].view(torch.int32).item())
    ws[12:16].zero_()
    assert err & 1, "error bit for a non-resident routed expert"
    assert_close(to_f32(out), ref["out"], what="layer output without the missing expert")


@pytest.mark.parametrize("name,T", [("c3_fp8", 2), ("c3_fp8", 9), ("c1_int8", 5), ("c2_gptq", 7), ("c3_full", 16),
                                    ("c3_fp8", 300)])
def test_negative_expert_ids_are_skipped(gpu, name, T):
    """Caller-supplied routing with id -1 for some pairs: those pairs contribute
    nothing (the combine skips their slots), no error bit is set, and the rest
    equals the oracle with those pairs' weights at zero.  c3_full is the full C3
    shape (the lean FP8 decode stages)."""
    from ftmoe.layer import workspace

    cfg = S.CONFIGS["c3_fp8"] if name == "c3_full" else S.SMALL[name]
    syn = S.generate(cfg, T=T, seed=70 + T)
    spec = oracle_spec(syn)
    rng = np.random.RandomState(T)
    ids = np.stack([rng.choice(syn.cfg.E, syn.cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
    w = O.round_bf16(rng.rand(T, syn.cfg.k).astype(np.float32))
    skip = rng.rand(T, syn.cfg.k) < 0.4
    skip[0, :] = True  # one token with no routed expert at all
    ref = O.layer_reference(spec, np_(syn.x), ids=ids, w=np.where(skip, 0.0, w).astype(np.float32))
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    ws = workspace(gpu, layer.workspace_bytes(T))
    ws[:16].zero_()
    ids_in = np.where(skip, -1, ids).astype(np.int32)
    out = layer.forward_routed(dsyn.x, torch.from_numpy(ids_in).to(gpu), torch.from_numpy(w).to(gpu))
    torch.cuda.synchronize()
    assert int(ws[12:16].view(torch.int32).item()) == 0, "no error bit for skipped pairs"
    assert_close(to_f32(out), ref["out"], what=f"{name} layer with skipped pairs")


@pytest.mark.parametrize("name,T", [("c1_int8", 3), ("c1_int8", 9), ("c2_gptq", 5), ("c4_mxfp4", 7),
                                    ("c3_nosh", 20), ("c3_full", 20)])
def test_call_with_no_routed_expert(gpu, name, T):
    """Caller routing whose every pair has no expert (a chunk past the last
    distinct expert of the device-LRU offload step), through each decode stage
    B (k_stage_b_xl at 3 tokens, k_stage_b_ks, k_stage_b_gq, k_stage_b_lean at
    20): no routed expert runs, every slot was zeroed by the top-k, and the
    output is exactly zero without a shared expert and the shared expert's
    contribution with one (c3_full)."""
    from dataclasses import replace

    if name == "c3_full":
        cfg = S.CONFIGS["c3_fp8"]
    elif name == "c3_nosh":
        cfg = replace(S.CONFIGS["c3_fp8"], shared_inter=0)
    else:
        cfg = S.SMALL[name]
    syn = S.generate(cfg, T=T, seed=130 + T)
    ids = np.full((T, syn.cfg.k), -1, np.int32)
    w = np.zeros((T, syn.cfg.k), np.float32)
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    for _ in range(2):  # the second call starts from the counters the first one left
        # a freed NaN block of the output's size: the caching allocator hands it
        # back as the output, so an output nobody writes shows up as NaN
        junk = torch.full((T, syn.cfg.H), float("nan"), dtype=dsyn.x.dtype, device=gpu)
        del junk
        out = layer.forward_routed(dsyn.x, ids_d, w_d)
        torch.cuda.synchronize()
        if syn.cfg.shared_inter == 0:
            assert torch.count_nonzero(out.float()).item() == 0, f"{name}: output not zero"
        else:
            ref = O.layer_reference(oracle_spec(syn), np_(syn.x), ids=ids, w=w)
            assert_close(to_f32(out), ref["out"], what=f"{name}: the shared expert alone")


@pytest.mark.parametrize("name,T", [("c3_fp8", 1), ("c3_fp8", 2), ("c3_fp8", 9), ("c3_fp8", 300), ("c3_full", 1),
                                    ("c3_full", 2), ("c2_gptq", 2)])
def test_repeated_expert_in_a_token_counts_twice(gpu, name, T):
    """Caller-supplied routing that lists one expert twice for a token applies it
    twice with both weights (the reference's per-expert loop,
    python/freetoken/kernel/triton/fused_moe.py:129-161, selects pairs by
    topk_ids == e).  At T = 1 and 2 the expert gets more pairs than there are
    tokens (T = 2: token 0 lists it twice, token 1 once), which the lists hold
    because a repeat's weight is folded into its first listing; no error bit.
    T=9 takes the one-workgroup-per-4-tokens top-k, T=300 the
    one-token-per-wave one; c3_full the lean decode stages."""
    from ftmoe.layer import read_status

    cfg = S.CONFIGS["c3_fp8"] if name == "c3_full" else S.SMALL[name]
    syn = S.generate(cfg, T=T, seed=90 + T)
    spec = oracle_spec(syn)
    rng = np.random.RandomState(T)
    ids = np.stack([rng.choice(syn.cfg.E, syn.cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
    e = int(ids[0, 0])
    ids[0, 1] = e
    if T >= 2:
        if e in ids[1]:  # token 1 lists e once, in column 2
            ids[1, ids[1].tolist().index(e)] = next(c for c in range(syn.cfg.E) if c != e and c not in ids[1])
        ids[1, 2] = e
        ids[T - 1, 3] = ids[T - 1, 2]
    w = O.round_bf16(rng.rand(T, syn.cfg.k).astype(np.float32))
    ref = O.layer_reference(spec, np_(syn.x), ids=ids, w=w)
    dsyn = syn.to(gpu)
    layer = S.build_layer(dsyn)
    read_status(gpu)
    out = layer.forward_routed(dsyn.x, torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu))
    assert read_status(gpu) == 0, "no error bit: every pair was applied"
    assert_close(to_f32(out), ref["out"], what="layer with a repeated expert")


def test_workspace_growth_keeps_captured_graphs_valid(gpu):
    """A HIP graph captured at T=8 keeps its workspace when a larger batch later
    grows the stream's workspace: replays after the growth still equal the
    eager result.  Growing inside a capture raises instead of allocating."""
    from ftmoe.layer import workspace

    syn = S.generate(S.SMALL["c3_fp8"], T=40, seed=31).to(gpu)
    layer = S.build_layer(syn)
    x8 = syn.x[:8].contiguous()
    ref8 = layer.forward(x8)
    ref40 = layer.forward(syn.x)
    s = torch.cuda.Stream(device=gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        layer.forward(x8)
        small = workspace(gpu, 0).data_ptr()
    torch.cuda.current_stream(gpu).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out8 = layer.forward(x8)
    with torch.cuda.stream(s):
        out40 = layer.forward(syn.x)  # grows this stream's workspace
        assert workspace(gpu, 0).data_ptr() != small
    torch.cuda.current_stream(gpu).wait_stream(s)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out8, ref8)
        layer.forward(syn.x)
        torch.cuda.synchronize()
    assert torch.equal(out40, ref40)
    # a capture that would have to grow the workspace refuses
    s2 = torch.cuda.Stream(device=gpu)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="inside a HIP graph capture"):
        with torch.cuda.graph(g2, stream=s2):
            layer.forward(x8)


def test_non_resident_expert_raises_when_checked(gpu):
    """forward_routed(check=True) turns the non-resident-slot error bit into
    IndexError (the reference's stale-slot tripwire,
    python/freetoken/models/qwen3_5_moe/__init__.py:1676-1685), and clears it."""
    from ftmoe.layer import check_status, read_status

    syn = S.generate(S.SMALL["c3_fp8"], T=3, seed=33)
    dsyn = syn.to(gpu)
    slots = torch.arange(syn.cfg.E, dtype=torch.int32, device=gpu)
    ids = torch.tensor([[0, 1, 2, 3]] * 3, dtype=torch.int32, device=gpu)[:, :syn.cfg.k]
    w = torch.full(ids.shape, 0.25, dtype=torch.float32, device=gpu)
    slots[1] = -1
    layer = S.build_layer(dsyn, slot_of_expert=slots)
    read_status(gpu)
    with pytest.raises(IndexError, match="stale slot map"):
        layer.forward_routed(dsyn.x, ids, w, check=True)
    assert read_status(gpu) == 0
    slots[1] = 1
    layer.forward_routed(dsyn.x, ids, w, check=True)
    check_status(gpu)


@pytest.mark.parametrize("mode", ["softmax_topk_lowp", "topk_softmax"])
@pytest.mark.parametrize("T", [1, 2, 3])
def test_c3_shape_route_modes(gpu, mode, T):
    """The C3 shape under the other two routing modes: T <= 2 routes inside
    the lean stage A (one instantiation per mode), T = 3 through the top-k
    kernel; routing bit-exact and outputs within tolerance either way."""
    from dataclasses import replace

    cfg = replace(S.CONFIGS["c3_fp8"], route_mode=mode)
    syn = S.generate(cfg, T=T, seed=60 + T)
    _run_and_check(syn, gpu)


# ---------------------------------------------------------------- router layouts
@pytest.mark.parametrize("E,shared,H,T", [
    (136, False, 2880, 16),  # k_route_topk1: one row per workgroup, rows in two load groups (6 chunk steps)
    (137, False, 320, 13),   # two rows per workgroup, the last one alone; a partial chunk step
    (272, True, 256, 9),     # 273 rows: four per workgroup, the shared-gate row in the last
    (40, False, 2880, 3),    # one row per workgroup, three of its waves busy
    (64, True, 2880, 1),     # one token
    (64, False, 1152, 20),   # k_router, one token per wave over five token blocks
    (300, True, 640, 40),    # k_router, four tokens per wave (301 x 10 blocks > 1300)
])
def test_router_layouts_bit_exact(gpu, E, shared, H, T):
    """Every layout the router kernels pick (rows per workgroup, tokens per
    wave, chunk steps per load group) keeps the fp32 summation order the
    oracle replays: logits, ids and weights bit-exact against it."""
    from ftmoe.banks import Proj
    from ftmoe.layer import MoeLayer

    I, k = 16, 4
    rng = np.random.RandomState(E + T)
    gate = O.f32_to_bf16_bits((rng.randn(E, H) * 0.05).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.randn(T, H).astype(np.float32))
    shd = None
    if shared:  # the shared-gate row rides in the router launch (rows = E + 1)
        sgate = O.f32_to_bf16_bits((rng.randn(1, H) * 0.05).astype(np.float32))
        shd = {"w13": torch.zeros(2 * I, H, dtype=torch.bfloat16, device=gpu),
               "w2": torch.zeros(H, I, dtype=torch.bfloat16, device=gpu),
               "gate": torch.from_numpy(sgate.view(np.int16)).view(torch.bfloat16).to(gpu)}
    w13 = Proj("bf16", torch.zeros(E, 2 * I, H, dtype=torch.bfloat16, device=gpu), 2 * I, H)
    w2 = Proj("bf16", torch.zeros(E, H, I, dtype=torch.bfloat16, device=gpu), H, I)
    g = torch.from_numpy(gate.view(np.int16)).view(torch.bfloat16).to(gpu)
    layer = MoeLayer(w13=w13, w2=w2, num_experts=E, hidden=H, inter=I, topk=k, gate_w=g, shared=shd,
                     act_dtype=torch.bfloat16)
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(gpu)
    out, ids, w, logits = layer.forward(xd, return_routing=True)
    torch.cuda.synchronize()
    ref_logits = O.router_logits(x, gate)
    rid, rw = O.route(ref_logits, k, "softmax_topk", True)
    kern = layer.stage_kernel(T, nat.STAGE_ROUTER)
    np.testing.assert_array_equal(to_f32(logits), ref_logits, err_msg=f"router logits ({kern})")
    np.testing.assert_array_equal(ids.cpu().numpy(), rid, err_msg=f"routing indices ({kern})")
    np.testing.assert_array_equal(w.cpu().numpy(), rw, err_msg=f"router weights ({kern})")
    assert torch.count_nonzero(out) == 0  # zero banks: only the routing is under test


# ---------------------------------------------------------------- LOWP routing on adversarial logits
def _route_only_layer(gpu, E, k, renorm, mode="softmax_topk_lowp"):
    from ftmoe.banks import Proj
    from ftmoe.layer import MoeLayer

    H, I = 64, 16
    w13 = Proj("bf16", torch.zeros(E, 2 * I, H, dtype=torch.bfloat16, device=gpu), 2 * I, H)
    w2 = Proj("bf16", torch.zeros(E, H, I, dtype=torch.bfloat16, device=gpu), H, I)
    return MoeLayer(w13=w13, w2=w2, num_experts=E, hidden=H, inter=I, topk=k, route_mode=mode,
                    renormalize=renorm, act_dtype=torch.bfloat16)


@pytest.mark.parametrize("E", [128, 256])
@pytest.mark.parametrize("T", [16, 100, 512])
@pytest.mark.parametrize("renorm", [True, False])
def test_lowp_routing_bit_exact_on_adversarial_logits(gpu, E, T, renorm):
    """LOWP routing (bf16 softmax, top-8 on bf16 probabilities) of caller
    logits through ftm_route, the fused backend's router: rows built so that
    a boundary probability sits within one fp32 ulp of a bf16 rounding
    midpoint or ties across the top-k boundary (tests/lowp_adversarial.py).
    Ids and weights equal the oracle's bit for bit at T = 16 (one-workgroup
    top-k), 100 (multi-workgroup) and 512 (one token per wave)."""
    from lowp_adversarial import adversarial_logits

    L = adversarial_logits(512, E, 8, seed=E)[:T]
    layer = _route_only_layer(gpu, E, 8, renorm)
    gating = torch.from_numpy(L).to(torch.bfloat16).to(gpu)
    ids, w, _ = layer.route(logits=gating)
    torch.cuda.synchronize()
    rid, rw = O.route(L, 8, "softmax_topk_lowp", renorm, weight_dt="bf16", prob_dt="bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), rid, err_msg="routing indices")
    np.testing.assert_array_equal(w.cpu().numpy(), rw, err_msg="router weights")


@pytest.mark.parametrize("mode", ["softmax_topk", "topk_softmax"])
def test_fp32_routing_weights_bit_exact_on_adversarial_logits(gpu, mode):
    """The fp32-softmax and gpt-oss modes on the same rows: every weight is
    one e^x, one lane-order sum and one division away from the logits, and
    equals the oracle's bit for bit."""
    from lowp_adversarial import adversarial_logits

    L = adversarial_logits(300, 128, 8, seed=7)
    layer = _route_only_layer(gpu, 128, 8, True, mode)
    ids, w, _ = layer.route(logits=torch.from_numpy(L).to(torch.bfloat16).to(gpu))
    torch.cuda.synchronize()
    rid, rw = O.route(L, 8, mode, True, weight_dt="bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_array_equal(w.cpu().numpy(), rw)


def test_fused_backend_on_adversarial_lowp_logits(gpu):
    """The fused backend end to end at the C2 router shape (128 experts,
    top-8) on the adversarial gating rows: output within tolerance of the
    oracle, whose routing it must reproduce to get there."""
    from lowp_adversarial import adversarial_logits
    from ftmoe.moe import create_moe_backend

    g = torch.Generator().manual_seed(3)
    E, H, I, T, K = 128, 256, 128, 256, 8
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gating = torch.from_numpy(adversarial_logits(T, E, K, seed=11)).to(torch.bfloat16)
    got = create_moe_backend("fused").forward(x.to(gpu), w1.to(gpu), w2.to(gpu), gating.to(gpu), K, True, "silu",
                                               False)
    ref = _fused_ref(x, w1, w2, gating, K, True, "silu", False, torch.bfloat16)
    assert_close(got.float().cpu().numpy(), ref, ATOL, RTOL, what="fused bf16, adversarial routing")


def _ks_layer(name, I, T, seed):
    """A small layer whose w2 rows need the K-split stage B (too long for one
    wave's window, short enough for a quarter of them): I = 2880 for MXFP4,
    1024 for INT8 and FP8; no shared expert."""
    from dataclasses import replace

    cfg = replace(S.SMALL[name], E=12, H=256, I=I, k=4, shared_inter=0)
    return S.generate(cfg, T=T, seed=seed)


@pytest.mark.parametrize("name,I,T", [("c4_mxfp4", 2880, 1), ("c4_mxfp4", 2880, 2), ("c1_int8", 1024, 2),
                                      ("c3_fp8", 1024, 1), ("c4_mxfp4", 2880, 3), ("c4_mxfp4", 2880, 5)])
def test_k_split_stage_b_with_combine(gpu, name, I, T):
    """Up to 8 routed experts (top-4: two tokens) the K-split stage B and the
    combine run as one launch (k_stage_bc_ks: one workgroup per 16 columns
    over every routed expert, the slot rows summed in LDS); above,
    k_stage_b_ks and k_combine.  Both against the oracle, for MXFP4 (with the
    gpt-oss biases), INT8 and FP8 rows."""
    layer, _, _, _ = _run_and_check(_ks_layer(name, I, T, 90 + T), gpu)
    fused = T <= 2
    assert layer.stage_kernel(T, nat.STAGE_W2) == ("k_stage_bc_ks" if fused else "k_stage_b_ks")
    assert layer.stage_kernel(T, nat.STAGE_COMBINE) == ("" if fused else "k_combine")


@pytest.mark.parametrize("T", [1, 2])
def test_k_split_stage_b_with_combine_skipped_and_missing(gpu, T):
    """k_stage_bc_ks with caller routing: pairs with id -1 contribute nothing,
    a routed expert without a slot contributes nothing and sets the error
    bit, and a second call on the same workspace gives the same output."""
    from ftmoe.layer import workspace

    syn = _ks_layer("c4_mxfp4", 2880, T, 120 + T)
    spec = oracle_spec(syn)
    ref_full = O.layer_reference(spec, np_(syn.x))
    ids = ref_full["ids"].astype(np.int32)
    w = ref_full["w"].astype(np.float32)
    missing = int(ids[0, 1])
    ids_in = ids.copy()
    ids_in[-1, -1] = -1  # one pair without an expert
    w_ref = np.where((ids == missing) | (ids_in < 0), 0.0, w).astype(np.float32)
    ref = O.layer_reference(spec, np_(syn.x), ids=ids, w=w_ref)
    dsyn = syn.to(gpu)
    slots = torch.arange(syn.cfg.E, dtype=torch.int32, device=gpu)
    slots[missing] = -1
    layer = S.build_layer(dsyn, slot_of_expert=slots)
    ws = workspace(gpu, layer.workspace_bytes(T))
    ws[:16].zero_()
    ids_d, w_d = torch.from_numpy(ids_in).to(gpu), torch.from_numpy(w).to(gpu)
    out = layer.forward_routed(dsyn.x, ids_d, w_d)
    torch.cuda.synchronize()
    err = int(ws[12:16].view(torch.int32).item())
    ws[12:16].zero_()
    assert err & 1, "error bit for a non-resident routed expert"
    assert_close(to_f32(out), ref["out"], what="k_stage_bc_ks without the missing expert and the skipped pair")
    again = layer.forward_routed(dsyn.x, ids_d, w_d)
    torch.cuda.synchronize()
    ws[12:16].zero_()
    assert torch.equal(out, again)


@pytest.mark.parametrize("name", ["c1_int8", "c4_mxfp4"])
def test_two_routed_experts_stage_b_with_combine(gpu, name):
    """One token on two experts of a layer whose w2 rows fit one wave's
    window: k_stage_bc_ks replaces k_stage_b_xl + k_combine (INT8 and MXFP4
    rows), against the oracle."""
    layer, _, _, _ = _run_and_check(S.generate(S.SMALL[name], T=1, seed=140), gpu)
    assert layer.stage_kernel(1, nat.STAGE_W2) == "k_stage_bc_ks"
    assert layer.stage_kernel(1, nat.STAGE_COMBINE) == ""
    assert layer.stage_kernel(2, nat.STAGE_W2) == "k_stage_b_xl"
