"""GPU: the offload slot pool (OffloadMoeCache + SlotWeightAccessor + the grouped
layer call over resident slots).

* copy_missing streams exactly the staged host rows into the staged slots
  (distinguishable banks, restating tests/test_moe_offload_cache.py:66-292);
* a two-layer FP8 pool smaller than one layer's experts: every decode step
  (route -> ensure_experts -> copy_missing -> moe_grouped_forward) matches the
  oracle computed from the full host bank, to the layer tolerance;
* a pool smaller than one step's routed experts (moe_offload_forward runs the
  step in chunks that fit) still computes every routed pair;
* SlotWeightAccessor.get is the bit-exact dequantization of the slot and
  expert_forward matches the oracle's expert."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import assert_close, np_, oracle_proj, oracle_spec, to_f32

from ftmoe import synthetic as S
from ftmoe.moe.offload_cache import OffloadMoeCache, SlotWeightAccessor, moe_grouped_forward, moe_offload_forward

pytestmark = pytest.mark.gpu

L, E, SL = 2, 4, 8
H, I = 16, 8


def _bank_values(layer, expert):
    base = 100 * (layer + 1) + 10 * (expert + 1)
    gate_up = torch.cat([torch.full((I, H), base + 0.0), torch.full((I, H), base + 1.0)])
    return gate_up, torch.full((H, I), base + 2.0)


def _sources():
    return {"gate_up": [torch.stack([_bank_values(l, e)[0] for e in range(E)]) for l in range(L)],
            "down": [torch.stack([_bank_values(l, e)[1] for e in range(E)]) for l in range(L)]}


def test_copy_missing_streams_the_staged_rows(gpu):
    c = OffloadMoeCache(L, E, E, gpu)
    c.set_bank_sources(_sources())
    c.materialize_layer(0)
    c.copy_missing()
    torch.cuda.synchronize()
    for e in range(E):
        gu, dn = _bank_values(0, e)
        assert torch.equal(c.bank_caches["gate_up"][e].cpu(), gu)
        assert torch.equal(c.bank_caches["down"][e].cpu(), dn)
    c.step.fill_(3)
    c.usage[:] = torch.arange(E, dtype=torch.int64) + 1
    c.ensure_experts(1, torch.tensor([0], device=gpu))  # evicts the LRU slot 0
    assert int(c.slot_for_id[1, 0]) == 0
    c.copy_missing()
    torch.cuda.synchronize()
    assert torch.equal(c.bank_caches["gate_up"][0].cpu(), _bank_values(1, 0)[0])
    assert torch.equal(c.bank_caches["down"][0].cpu(), _bank_values(1, 0)[1])
    for e in range(1, E):  # untouched slots keep layer 0
        assert torch.equal(c.bank_caches["down"][e].cpu(), _bank_values(0, e)[1])
    sl = c.slot_of_expert(1)
    assert sl.is_cuda and sl.dtype == torch.int32 and sl.tolist() == [0, -1, -1, -1]


def _fp8_pool(gpu, slots, seeds=(31, 32)):
    cfg = S.SMALL["c3_fp8"]
    syns = [S.generate(cfg, T=12, seed=s) for s in seeds]
    c = OffloadMoeCache(len(syns), cfg.E, slots, gpu, quant_format="fp8_block", decode_only=slots < cfg.E)
    c.set_bank_sources({b: [syn.bank[b] for syn in syns] for b in c.bank_schema})
    return cfg, syns, c


def test_fp8_pool_decode_steps_match_oracle(gpu):
    cfg, syns, c = _fp8_pool(gpu, slots=24)  # 24 slots for 2 layers x 32 experts (decode-only pool)
    rng = np.random.RandomState(5)
    T = 5  # at most 20 routed experts per step: all of them fit the 24 slots at once
    for step in range(6):
        layer_id = step % 2
        syn = syns[layer_id]
        x = syn.x[:T]
        ids = np.stack([rng.choice(cfg.E, cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
        w = O.round_bf16(rng.rand(T, cfg.k).astype(np.float32))
        c.ensure_experts(layer_id, torch.from_numpy(ids).to(gpu))
        c.copy_missing()
        shared = {k: v.to(gpu) for k, v in syn.shared.items()}
        out = moe_grouped_forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), c,
                                  layer_id, intermediate=cfg.I, shared=shared)
        ref = O.layer_reference(oracle_spec(syn), np_(x), ids=ids, w=w)
        assert_close(to_f32(out), ref["out"], what=f"pool step {step}")
    st = c.decode_miss_stats()
    assert st["calls"] == 6 and st["missing"] > 0


def test_steps_with_more_experts_than_slots_run_in_chunks(gpu):
    cfg, syns, c = _fp8_pool(gpu, slots=6)  # 6 slots; T=5 x top-4 routes up to 20 experts
    rng = np.random.RandomState(9)
    T = 5
    chunked = 0
    for step in range(4):
        layer_id = step % 2
        syn = syns[layer_id]
        x = syn.x[:T]
        ids = np.stack([rng.choice(cfg.E, cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
        w = O.round_bf16(rng.rand(T, cfg.k).astype(np.float32))
        chunked += len(np.unique(ids)) > 6
        shared = {k: v.to(gpu) for k, v in syn.shared.items()}
        out = moe_offload_forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), c,
                                  layer_id, intermediate=cfg.I, shared=shared)
        ref = O.layer_reference(oracle_spec(syn), np_(x), ids=ids, w=w)
        assert_close(to_f32(out), ref["out"], what=f"chunked pool step {step}")
    assert chunked == 4


def test_accessor_get_and_expert_forward(gpu):
    cfg, syns, c = _fp8_pool(gpu, slots=32, seeds=(33,))
    c.materialize_layer(0)
    c.copy_missing()
    acc = SlotWeightAccessor(c, cfg.I, torch.bfloat16)
    spec13 = oracle_proj(cfg.fmt, syns[0].bank, "gate_up", 2 * cfg.I, cfg.H, cfg.group)
    spec2 = oracle_proj(cfg.fmt, syns[0].bank, "down", cfg.H, cfg.I, cfg.group)
    g = torch.Generator().manual_seed(7)
    x_many = torch.randn(40, cfg.H, generator=g).to(torch.bfloat16)
    for slot in (0, 5, 31):
        e = int(c.id_of_slot[slot]) % cfg.E
        gate, up, down = acc.get(slot)
        gu_ref = O.round_bf16(O.dequant(spec13, e))
        np.testing.assert_array_equal(to_f32(gate), gu_ref[:cfg.I])
        np.testing.assert_array_equal(to_f32(up), gu_ref[cfg.I:])
        np.testing.assert_array_equal(to_f32(down), O.round_bf16(O.dequant(spec2, e)))
        # 3 rows: below the FP8 crossover (8); 40 rows: above it, where the
        # reference dequantizes and the expert runs on the tiled HIP stages
        for x in (syns[0].x[:3], x_many):
            got = acc.expert_forward(slot, x.to(gpu))
            ref = O.expert_forward(spec13, spec2, e, O.bf16_bits_to_f32(np_(x)))
            assert_close(to_f32(got), ref, what=f"expert slot {slot}, {x.shape[0]} rows")
    fp8 = acc.get_fp8_packed(0)
    assert fp8[0].shape == (2 * cfg.I, cfg.H) and fp8[4] == 128


def _zipf_steps(E, T, k, steps, seed):
    """C5 routing: per token k distinct experts drawn Zipf(1.1) over ranks mapped
    through a seeded permutation; weights the softmax of N(0, 1) logits, bf16."""
    rng = np.random.RandomState(seed)
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([np.stack([perm[rng.choice(E, k, replace=False, p=p)] for _ in range(T)])
                    for _ in range(steps)]).astype(np.int32)
    z = rng.randn(steps, T, k)
    w = np.exp(z - z.max(-1, keepdims=True))
    return ids, O.round_bf16((w / w.sum(-1, keepdims=True)).astype(np.float32))


@pytest.mark.parametrize("device_lru", [True, False])
def test_c5_offload_full_shape_matches_oracle(gpu, device_lru):
    """C5 at its own shape: the C3 FP8 layer (256 experts, H=2048, I=512, top-8,
    shared expert) with 64 HBM slots fed from pinned host banks, 16-token
    decode steps with Zipf routing.  Steps 0 and 2 route to more than 64
    experts (67 and 65) and run in chunks.  Every step's output matches the
    oracle on the full bank."""
    cfg = S.CONFIGS["c3_fp8"]
    syn = S.generate(cfg, T=16, seed=5, device=gpu)
    host = syn.to("cpu")
    ids_all, w_all = _zipf_steps(cfg.E, 16, cfg.k, 4, seed=3)
    distinct = [len(np.unique(s)) for s in ids_all]
    assert max(distinct) > 64 and min(distinct) <= 64, distinct
    c = OffloadMoeCache(1, cfg.E, 64, gpu, quant_format="fp8_block", decode_only=True, device_lru=device_lru)
    c.set_bank_sources({b: [host.bank[b]] for b in c.bank_schema})
    spec = oracle_spec(host)
    g = torch.Generator().manual_seed(55)
    for step in range(4):
        x = torch.randn(16, cfg.H, generator=g).to(torch.bfloat16)
        print(f"c5 full shape device_lru={device_lru} step {step} distinct={distinct[step]}", flush=True)
        out = moe_offload_forward(x.to(gpu), torch.from_numpy(ids_all[step]).to(gpu),
                                  torch.from_numpy(w_all[step]).to(gpu), c, 0, intermediate=cfg.I, shared=syn.shared)
        ref = O.layer_reference(spec, np_(x), ids=ids_all[step], w=w_all[step])
        assert_close(to_f32(out), ref["out"], what=f"C5 step {step} ({distinct[step]} experts)")
    c.check_status()
    assert c.decode_miss_stats()["missing"] > 0
