"""C ABI on the CPU: the library loads, exports exactly what include/ftmoe.h
declares, and rejects bad arguments with the reference's error convention
(python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:733-739) before touching
the HIP runtime, so every error path is exercised without a GPU."""
import ctypes
import os
import re

import pytest

from ftmoe import _native as nat

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "ftmoe.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ftm_[a-z0-9_]+)\s*\(", src)))


def test_exports_match_header():
    L = nat.lib()
    declared = _declared()
    assert declared == sorted(nat.EXPORTED)
    for name in declared:
        assert hasattr(L, name), name
    assert L.ftm_version() == nat.ABI_VERSION


def _proj(**kw):
    p = nat.FtmProj()
    p.w = kw.get("w", 0x1000)
    p.s = kw.get("s", 0x2000)
    p.z = kw.get("z", None)
    p.fmt = kw.get("fmt", nat.FMT_FP8_BLOCK)
    p.s_dtype = nat.DT_F32
    p.group = kw.get("group", 128)
    p.N = kw.get("N", 256)
    p.K = kw.get("K", 256)
    p.num_slots = kw.get("num_slots", 1)
    return p


def test_linear_argument_errors():
    L = nat.lib()
    x = ctypes.c_void_p(0x4000)
    out = ctypes.c_void_p(0x8000)

    def call(p, slot=0, M=4, xx=x, oo=out, dt=nat.DT_F32):
        return L.ftm_linear(ctypes.byref(p) if p is not None else None, slot, xx, dt, M, oo, dt, None, 0, dt, None)

    assert call(None) == nat.ERR_NULL
    assert call(_proj(w=None)) == nat.ERR_NULL
    assert call(_proj(s=None)) == nat.ERR_NULL
    assert call(_proj(N=0)) == nat.ERR_DIM
    assert call(_proj(fmt=99)) == nat.ERR_FORMAT
    assert call(_proj(), slot=1) == nat.ERR_DIM
    assert call(_proj(), M=-1) == nat.ERR_DIM
    assert call(_proj(), M=0) == nat.OK  # empty batch is a no-op
    assert call(_proj(), xx=None) == nat.ERR_NULL
    assert call(_proj(), dt=7) == nat.ERR_FORMAT
    assert call(_proj(fmt=nat.FMT_GPTQ_INT4, z=None)) == nat.ERR_NULL


def _layer(**kw):
    L = nat.FtmMoeLayer()
    L.w13 = _proj(N=2 * kw.get("I", 128), K=kw.get("H", 256), num_slots=8)
    L.w2 = _proj(N=kw.get("H", 256), K=kw.get("I", 128), num_slots=8)
    L.num_experts = kw.get("E", 8)
    L.hidden = kw.get("H", 256)
    L.inter = kw.get("I", 128)
    L.topk = kw.get("k", 2)
    L.gate_w = kw.get("gate_w", 0x9000)
    L.act_dtype = kw.get("act_dtype", nat.DT_BF16)
    L.route_mode = kw.get("route_mode", nat.ROUTE_SOFTMAX_TOPK)
    L.act = kw.get("act", nat.ACT_SILU)
    return L


def test_layer_argument_errors():
    lib = nat.lib()
    x, out, ws = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000), ctypes.c_void_p(0x40000)

    def fwd(L, T=4, wsb=1 << 30, wsp=ws):
        return lib.ftm_moe_forward(ctypes.byref(L), x, T, out, None, None, None, wsp, wsb, None)

    assert fwd(_layer(E=0)) == nat.ERR_DIM
    assert fwd(_layer(k=9)) == nat.ERR_DIM  # k > E
    assert fwd(_layer(E=600, k=2)) == nat.ERR_DIM
    assert fwd(_layer(gate_w=None)) == nat.ERR_NULL
    assert fwd(_layer(act_dtype=nat.DT_F16)) == nat.ERR_FORMAT
    assert fwd(_layer(route_mode=9)) == nat.ERR_FORMAT
    assert fwd(_layer(act=9)) == nat.ERR_FORMAT
    assert fwd(_layer(), T=-1) == nat.ERR_DIM
    assert fwd(_layer(), T=0) == nat.OK
    assert fwd(_layer(), wsp=None) == nat.ERR_WORKSPACE
    assert fwd(_layer(), wsb=16) == nat.ERR_WORKSPACE
    assert fwd(_layer(), wsp=ctypes.c_void_p(0x40010)) == nat.ERR_ALIGN
    bad = _layer()
    bad.w2.K = 64  # w2 must be [H, I]
    assert fwd(bad) == nat.ERR_DIM
    assert lib.ftm_moe_workspace_bytes(ctypes.byref(_layer()), 4) > nat.WS_CTRL_BYTES


def test_copy_slots_argument_errors():
    lib = nat.lib()
    ev = (ctypes.c_int32 * 2)(0, 1)
    assert lib.ftm_copy_slots(None, None, 64, None, None, -1, None, None) == nat.ERR_DIM
    assert lib.ftm_copy_slots(None, None, 0, None, None, 0, None, None) == nat.ERR_DIM
    assert lib.ftm_copy_slots(None, None, 64, ev, ev, 2, None, None) == nat.ERR_NULL
    neg = (ctypes.c_int32 * 1)(-1)
    assert lib.ftm_copy_slots(ctypes.c_void_p(16), ctypes.c_void_p(32), 64, neg, ev, 1, None, None) == nat.ERR_DIM


def test_device_lru_and_copy_argument_errors():
    lib = nat.lib()
    p = ctypes.c_void_p(0x1000)

    def ens(L=2, E=8, S=4, layer=0, n=3, chunk=0, cap=8, ids=p, sfi=p):
        return lib.ftm_lru_ensure_dev(layer, L, E, S, ids, n, chunk, cap, sfi, p, p, p, p, p, p, None, None, None,
                                      None)

    assert ens(E=0) == nat.ERR_DIM
    assert ens(E=513) == nat.ERR_DIM  # one expert per thread of the workgroup
    assert ens(S=0) == nat.ERR_DIM
    assert ens(S=(1 << 21) + 1) == nat.ERR_DIM  # slot index packed in 21 bits
    assert ens(layer=2) == nat.ERR_DIM
    assert ens(n=-1) == nat.ERR_DIM
    assert ens(chunk=-1) == nat.ERR_DIM
    assert ens(cap=0) == nat.ERR_DIM
    assert ens(ids=None) == nat.ERR_NULL
    assert ens(sfi=None) == nat.ERR_NULL
    B = nat.FtmBankCopy
    one = (B * 1)(B(0x1000, 0x2000, 64))

    def cp(banks=one, nb=1, rows=4, slots=4, ev=p, mx=2):
        return lib.ftm_copy_slots_dev(banks, nb, rows, slots, ev, p, p, mx, None)

    assert cp(nb=0) == nat.ERR_DIM
    assert cp(nb=9) == nat.ERR_DIM
    assert cp(rows=0) == nat.ERR_DIM
    assert cp(slots=0) == nat.ERR_DIM
    assert cp(mx=-1) == nat.ERR_DIM
    assert cp(banks=None) == nat.ERR_NULL
    assert cp(ev=None) == nat.ERR_NULL
    assert cp(banks=(B * 1)(B(0x1000, 0x2000, 0))) == nat.ERR_DIM
    assert cp(banks=(B * 1)(B(None, 0x2000, 64))) == nat.ERR_NULL
    assert cp(mx=0) == nat.OK  # nothing to copy: no launch


def test_stage_kernel_names_follow_the_dispatch():
    """ftm_moe_stage_kernel names the kernel each stage launches: the lean FP8
    decode stages for the 2048x512 shape below the token crossover, the tiled
    GEMM stages at >= 16 tokens per routed expert, the LDS-activation stages
    up to 4 tokens and the register-fed ones above for other shapes."""
    lib = nat.lib()

    def name(L, T, st):
        r = lib.ftm_moe_stage_kernel(ctypes.byref(L), T, st)
        return r.decode() if r is not None else None

    c3 = _layer(E=256, H=2048, I=512, k=8)
    c3.shared_inter, c3.shared_w13, c3.shared_w2, c3.shared_gate = 512, 0xA0000, 0xB0000, 0xC0000
    for T in (1, 2):  # small batches route inside stage A: the top-k stage launches nothing
        assert name(c3, T, nat.STAGE_W13) == "k_stage_a_lean_route", T
        assert name(c3, T, nat.STAGE_TOPK) == "", T
    for T in (3, 4, 16, 64, 256):
        assert name(c3, T, nat.STAGE_W13) == "k_stage_a_lean", T
    for T in (1, 4, 16):  # stage B and the combine in one launch
        assert name(c3, T, nat.STAGE_W2) == "k_stage_bc_lean", T
        assert name(c3, T, nat.STAGE_COMBINE) == "", T
    for T in (17, 64, 256):
        assert name(c3, T, nat.STAGE_W2) == "k_stage_b_lean", T
    # 512 tokens x top-8 = 16 pairs per expert on all 256 experts: GEMM
    # stages, the routed experts on the scaled-MFMA tiles (FP8 128 x 128 blocks)
    assert name(c3, 512, nat.STAGE_W13) == "k_gemm_mx"
    # stage B: I = 512 (a multiple of 128 up to 512) keeps the tile's h rows
    # in LDS and feeds the weights from registers; I = 640 takes the ring tile
    assert name(c3, 512, nat.STAGE_W2) == "k_gemm_mxb_f8"
    wide = _layer(E=256, H=2048, I=640, k=8)
    assert name(wide, 512, nat.STAGE_W2) == "k_gemm_mx"
    c3.w2.flags = nat.PROJ_RING_B  # the ring tile on request (tests compare the two)
    assert name(c3, 512, nat.STAGE_W2) == "k_gemm_mx"
    c3.w2.flags = 0
    # the GPU test's shapes (32 experts, top-4, 512 tokens) reach the register-fed tile
    for H, I in ((384, 384), (256, 128), (256, 256), (640, 512)):
        Ls = _layer(E=32, H=H, I=I, k=4)
        assert name(Ls, 512, nat.STAGE_W2) == "k_gemm_mxb_f8", (H, I)
    assert name(_layer(E=32, H=320, I=384, k=4), 512, nat.STAGE_W2) == "k_gemm_b"  # H % 128 != 0
    # 3..16 tokens: router and top-k in one launch (the top-k stage launches nothing)
    for T in (3, 16):
        assert name(c3, T, nat.STAGE_ROUTER) == "k_route_topk1", T
        assert name(c3, T, nat.STAGE_TOPK) == "", T
    assert name(c3, 17, nat.STAGE_TOPK) == "k_topk"
    assert name(c3, 255, nat.STAGE_TOPK) == "k_topk"
    assert name(c3, 256, nat.STAGE_TOPK) == "k_topk_blk"
    assert name(c3, 17, nat.STAGE_ROUTER) == "k_router"
    # k_router_rows once k_router would re-read x more than 40 M elements (rows x T x H)
    assert name(c3, 64, nat.STAGE_ROUTER) == "k_router"
    assert name(c3, 128, nat.STAGE_ROUTER) == "k_router_rows"
    assert name(c3, 17, nat.STAGE_COMBINE) == "k_combine"
    assert name(c3, 16, 5) is None
    assert name(c3, 0, nat.STAGE_W13) is None
    small = _layer(E=8, H=256, I=128, k=2)
    assert name(small, 4, nat.STAGE_W13) == "k_stage_a_xl"
    assert name(small, 4, nat.STAGE_ROUTER) == "k_router"  # routed inside k_stage_a_xl
    assert name(small, 4, nat.STAGE_TOPK) == ""
    assert name(small, 5, nat.STAGE_ROUTER) == "k_route_topk1"
    c1 = _layer(E=16, H=1024, I=512, k=2)  # INT8 per-channel, C1's shape
    c1.w13 = _proj(N=1024, K=1024, num_slots=16, fmt=nat.FMT_INT8_PACKED, group=1024)
    c1.w2 = _proj(N=1024, K=512, num_slots=16, fmt=nat.FMT_INT8_PACKED, group=512)
    assert name(c1, 4, nat.STAGE_W13) == "k_stage_a_xl"
    assert name(c1, 4, nat.STAGE_ROUTER) == "k_router"
    assert name(c1, 4, nat.STAGE_TOPK) == ""
    assert name(small, 4, nat.STAGE_W2) == "k_stage_b_xl"
    assert name(small, 1, nat.STAGE_W2) == "k_stage_bc_ks"  # two routed experts: stage B with the combine
    assert name(small, 1, nat.STAGE_COMBINE) == ""
    assert name(small, 5, nat.STAGE_W13) == "k_stage_a_rows"
    assert name(small, 5, nat.STAGE_W2) == "k_stage_b_ks"  # K split over the waves up to 32 tokens
    assert name(small, 33, nat.STAGE_W2) == "k_stage_b"
    assert name(small, 64, nat.STAGE_W13) == "k_gemm_mx"  # FP8 128 x 128 blocks: scaled-MFMA tiles
    # GPTQ group 128: activation rows in LDS up to 16 tokens while half of the
    # hidden size fits a wave's K range (1024), the register-fed kernel above
    gq = _layer(E=128, H=2048, I=768, k=8)
    gq.w13 = _proj(N=2 * 768, K=2048, num_slots=8, fmt=nat.FMT_GPTQ_INT4, z=0x3000)
    gq.w2 = _proj(N=2048, K=768, num_slots=8, fmt=nat.FMT_GPTQ_INT4, z=0x3000)
    for T in (1, 4, 16):
        assert name(gq, T, nat.STAGE_W13) == "k_stage_a_gq", T
        assert name(gq, T, nat.STAGE_W2) == "k_stage_b_gq", T
    for T in (1, 2, 4):  # k_stage_a_gq routes the tokens itself: no top-k launch
        assert name(gq, T, nat.STAGE_ROUTER) == "k_router", T
        assert name(gq, T, nat.STAGE_TOPK) == "", T
    for T in (5, 16):
        assert name(gq, T, nat.STAGE_ROUTER) == "k_route_topk1", T
        assert name(gq, T, nat.STAGE_TOPK) == "", T
    assert name(gq, 17, nat.STAGE_W13) == "k_stage_a"
    assert name(gq, 32, nat.STAGE_W2) == "k_stage_b_gq"  # stage B keeps LDS rows up to 32 tokens
    assert name(gq, 33, nat.STAGE_W2) == "k_stage_b"
    gq.hidden = 2176  # 17 groups: a wave's half would be 1152 wide
    gq.w13.K, gq.w2.N = 2176, 2176
    assert name(gq, 4, nat.STAGE_W13) == "k_stage_a"
    # MXFP4 (C4 shape): stage A on scaled MFMAs with activations in LDS and
    # stage B with w2's 2880-wide K split over the waves below 4 tokens per
    # expert, the token-resident stages from 4 up to 16 (T = 128 on 32
    # experts, top-4); the GEMM tiles above
    mx = _layer(E=32, H=2880, I=2880, k=4)
    mx.w13 = _proj(N=2 * 2880, K=2880, num_slots=8, fmt=nat.FMT_MXFP4, group=32)
    mx.w2 = _proj(N=2880, K=2880, num_slots=8, fmt=nat.FMT_MXFP4, group=32)
    for T in (1, 8, 31):
        assert name(mx, T, nat.STAGE_W13) == "k_stage_a_xl", T
    for T in (1, 2):  # up to 8 routed experts stage B and the combine run as one launch
        assert name(mx, T, nat.STAGE_W2) == "k_stage_bc_ks", T
        assert name(mx, T, nat.STAGE_COMBINE) == "", T
    for T in (3, 5, 8, 31):
        assert name(mx, T, nat.STAGE_W2) == "k_stage_b_ks", T
        assert name(mx, T, nat.STAGE_COMBINE) == "k_combine", T
    for T in (32, 64, 128):  # 4 to 16 tokens per expert: token rows resident in LDS, both stages
        assert name(mx, T, nat.STAGE_W13) == "k_stage_tok_a", T
        assert name(mx, T, nat.STAGE_W2) == "k_stage_tok_b", T
    # one token: k_stage_a_xl routes it (4 experts x 360 items fit one round of
    # workgroups); two tokens' 2880 items would not, so they keep the top-k
    assert name(mx, 1, nat.STAGE_ROUTER) == "k_router"
    assert name(mx, 1, nat.STAGE_TOPK) == ""
    assert name(mx, 2, nat.STAGE_ROUTER) == "k_route_topk1"
    assert name(mx, 128, nat.STAGE_ROUTER) == "k_router"  # 32 rows: one row per workgroup
    assert name(mx, 512, nat.STAGE_ROUTER) == "k_router_rows"
    assert name(mx, 129, nat.STAGE_W13) == "k_gemm_mx"  # scaled-MFMA tiles (no shared expert)
    assert name(mx, 129, nat.STAGE_W2) == "k_gemm_mx"
    # many experts: the LDS path up to 256 tokens, the register-fed kernels above
    mx.num_experts = 256
    assert name(mx, 200, nat.STAGE_W13) == "k_stage_a_xl"  # about 3 tokens per expert
    assert name(mx, 200, nat.STAGE_W2) == "k_stage_b_ks"
    assert name(mx, 256, nat.STAGE_W13) == "k_stage_tok_a"  # 4 per expert
    assert name(mx, 256, nat.STAGE_W2) == "k_stage_tok_b"
    assert name(mx, 257, nat.STAGE_W13) == "k_stage_a_rows"
    assert name(mx, 257, nat.STAGE_W2) == "k_stage_b"
    f32 = _layer(E=8, H=256, I=128, k=2, act_dtype=nat.DT_F32)
    assert name(f32, 4, nat.STAGE_W13) is None  # f32 activations need the bf16 router: invalid layer
