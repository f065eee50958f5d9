"""GPU: the engine-side MoE block (ftmoe.engine.MoeBlock, the grouped
replacement of _Qwen35MoE.forward / _Qwen3MoE.forward and their per-pair
offload loop) against the oracle, and decode steps captured in HIP graphs
(MoeGraphRunner, the analogue of XpuGraphRunner) replaying to the eager
result -- for the in-HBM block and for an offload block whose LRU and copies
run on the GPU, whose pool state must evolve exactly as an eager twin's."""
from dataclasses import replace

import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import assert_close, np_, oracle_spec, to_f32

from ftmoe import synthetic as S
from ftmoe.banks import proj_from_bank
from ftmoe.engine import MoeBlock, MoeGraphRunner
from ftmoe.moe.offload_cache import OffloadMoeCache

pytestmark = pytest.mark.gpu


def _block(syn, gpu, *, softmax_fp32=True, cache=None):
    cfg = syn.cfg
    Is = cfg.shared_inter
    sh = syn.shared
    shared = (sh["w13"][:Is], sh["w13"][Is:], sh["w2"], sh["gate"]) if sh is not None else None
    if cache is None:
        w13 = proj_from_bank(cfg.fmt, syn.bank, which="gate_up", N=2 * cfg.I, K=cfg.H, group=cfg.group)
        w2 = proj_from_bank(cfg.fmt, syn.bank, which="down", N=cfg.H, K=cfg.I, group=cfg.group)
        return MoeBlock(gate=syn.gate_w, top_k=cfg.k, intermediate=cfg.I, softmax_fp32=softmax_fp32, shared=shared,
                        w13=w13, w2=w2)
    return MoeBlock(gate=syn.gate_w, top_k=cfg.k, intermediate=cfg.I, softmax_fp32=softmax_fp32, shared=shared,
                    cache=cache, layer_id=0)


@pytest.mark.parametrize("mode", ["softmax_topk", "softmax_topk_lowp"])
def test_block_matches_oracle(gpu, mode):
    cfg = replace(S.SMALL["c3_fp8"], route_mode=mode)
    syn = S.generate(cfg, T=6, seed=400).to(gpu)
    block = _block(syn, gpu, softmax_fp32=mode == "softmax_topk")
    x3 = syn.x.reshape(2, 3, cfg.H)  # [batch, seq, hidden] in, same shape out
    out = block(x3)
    assert out.shape == x3.shape
    ref = O.layer_reference(oracle_spec(syn), np_(syn.x))
    assert_close(to_f32(out.reshape(6, cfg.H)), ref["out"], what=f"MoE block ({mode})")


def test_graph_replays_equal_eager(gpu):
    syn = S.generate(S.SMALL["c3_fp8"], T=8, seed=401).to(gpu)
    block = _block(syn, gpu)
    static_x = syn.x.clone()
    static_out = torch.empty_like(static_x)
    runner = MoeGraphRunner()
    runner.capture(lambda: static_out.copy_(block(static_x)))
    g = torch.Generator(device=gpu).manual_seed(5)
    for i in range(4):
        x = torch.randn(8, syn.cfg.H, generator=g, device=gpu).to(torch.bfloat16)
        static_x.copy_(x)
        runner.replay()
        ref = block(x)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static_out, ref), i


def test_offload_decode_step_captured_with_device_lru(gpu):
    """The whole offload decode step -- router, device LRU, copy kernel from the
    pinned banks, grouped layer (in chunks: 32 distinct experts can exceed the
    12 slots) -- captured once and replayed; every replay equals an eager twin
    pool's step on the same input and leaves the same LRU state."""
    cfg = S.SMALL["c3_fp8"]
    syn = S.generate(cfg, T=6, seed=402)
    dsyn = syn.to(gpu)

    def pool():
        c = OffloadMoeCache(1, cfg.E, 12, gpu, quant_format="fp8_block", decode_only=True, device_lru=True)
        c.set_bank_sources({b: [syn.bank[b]] for b in c.bank_schema})
        return c

    cg, ce = pool(), pool()
    bg, be = _block(dsyn, gpu, cache=cg), _block(dsyn, gpu, cache=ce)
    static_x = dsyn.x.clone()
    static_out = torch.empty_like(static_x)
    runner = MoeGraphRunner(warmup_iters=2)
    runner.capture(lambda: static_out.copy_(bg(static_x)))
    for _ in range(2):  # the twin takes the runner's warm-up steps
        be(dsyn.x)
    g = torch.Generator(device=gpu).manual_seed(6)
    spec = oracle_spec(syn)
    for i in range(4):
        x = torch.randn(6, cfg.H, generator=g, device=gpu).to(torch.bfloat16)
        static_x.copy_(x)
        runner.replay()
        ref = be(x)
        torch.cuda.synchronize()
        assert torch.equal(static_out, ref), i
        assert cg.id_of_slot.tolist() == ce.id_of_slot.tolist() and cg.usage.tolist() == ce.usage.tolist(), i
        oref = O.layer_reference(spec, np_(x))
        assert_close(to_f32(static_out), oref["out"], what=f"captured offload step {i}")
    cg.check_status()
    ce.check_status()
