"""GPU: the hybrid CPU || GPU decode step (ftmoe.moe.hybrid.moe_hybrid_forward,
restating python/freetoken/models/qwen3_moe/__init__.py:679-866): for every
bank format, the routed experts split between the host CPU kernel
(ftm_cpu_moe_forward on the pool's pinned host banks) and the GPU slot pool,
summed, match the oracle on the full bank -- at several fetch fractions, with
the host and the device LRU, and with the gpt-oss MXFP4 biases riding in the
slots.  The CPU half keeps h in fp32 and the GPU half rounds it to bf16; both
are within the layer tolerance of the oracle's bf16-h layer."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import assert_close, np_, oracle_spec, to_f32

from ftmoe import synthetic as S
from ftmoe.moe import hybrid as HY
from ftmoe.moe.offload_cache import OffloadMoeCache

pytestmark = pytest.mark.gpu

NAMES = ["c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"]


def _pool(name, gpu, *, slots, device_lru, seed):
    cfg = S.SMALL[name]
    syn = S.generate(cfg, T=8, seed=seed)
    c = OffloadMoeCache(1, cfg.E, slots, gpu, quant_format=cfg.fmt, decode_only=slots < cfg.E, device_lru=device_lru)
    src = {b: [syn.bank[b]] for b in syn.bank}
    if syn.bias13 is not None:
        src["bias_gate_up"], src["bias_down"] = [syn.bias13], [syn.bias2]
    c.set_bank_sources(src)
    if cfg.fmt == "gptq_int4":
        c.gptq_group_size = cfg.group
    elif cfg.fmt == "int8_channel":
        c.int8_k_gate_up, c.int8_k_down = cfg.H, cfg.I
    elif cfg.fmt == "fp8_block":
        c.fp8_block_size = cfg.group
    return cfg, syn, c


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("device_lru", [False, True])
def test_hybrid_steps_match_oracle(gpu, name, device_lru):
    cfg, syn, c = _pool(name, gpu, slots=max(8, cfg_slots(name)), device_lru=device_lru, seed=600)
    spec = oracle_spec(syn)
    shared = {k: v.to(gpu) for k, v in syn.shared.items()} if syn.shared is not None else None
    rng = np.random.RandomState(17)
    for step, f in enumerate((0.25, 0.5, 0.75, 0.5)):
        T = 3 + step
        x = syn.x[:T] if T <= syn.x.shape[0] else syn.x.repeat(2, 1)[:T]
        ids = np.stack([rng.choice(cfg.E, cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
        w = O.round_bf16(rng.rand(T, cfg.k).astype(np.float32))
        print(f"hybrid {name} device_lru={device_lru} step {step} f={f} T={T}", flush=True)
        cpu_set = HY.split_experts(torch.from_numpy(ids), f)
        assert cpu_set and len(cpu_set) < len(np.unique(ids))
        out = HY.moe_hybrid_forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), c, 0,
                                    intermediate=cfg.I, fetch_fraction=f, act=cfg.act, shared=shared,
                                    swiglu_alpha=cfg.swiglu_alpha, swiglu_limit=cfg.swiglu_limit)
        ref = O.layer_reference(spec, np_(x), ids=ids, w=w)
        assert out.dtype == x.dtype and out.shape == x.shape
        assert_close(to_f32(out), ref["out"], what=f"{name} hybrid step {step} (f={f})")
        # the CPU's experts never entered the pool on this step
        resident = set(c.slot_for_id[0].cpu().ge(0).nonzero().flatten().tolist())
        assert not (cpu_set & resident) or step > 0
    c.check_status()


def cfg_slots(name):
    """A pool smaller than the layer (decode-only) where the layer allows it."""
    return S.SMALL[name].E // 2


def test_hybrid_with_nothing_to_split_is_the_offload_step(gpu):
    cfg, syn, c = _pool("c3_fp8", gpu, slots=32, device_lru=False, seed=601)
    x = syn.x[:1]
    ids = np.array([[3, 9, 1, 30]], np.int32)
    w = O.round_bf16(np.array([[0.4, 0.3, 0.2, 0.1]], np.float32))
    shared = {k: v.to(gpu) for k, v in syn.shared.items()}
    for f in (0.0, 1.0):
        out = HY.moe_hybrid_forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), c, 0,
                                    intermediate=cfg.I, fetch_fraction=f, shared=shared)
        ref = O.layer_reference(oracle_spec(syn), np_(x), ids=ids, w=w)
        assert_close(to_f32(out), ref["out"], what=f"no split (f={f})")
