"""Slot-pool bookkeeping of OffloadMoeCache on the host (no GPU needed).

The cases restate the reference's own LRU tests (tests/test_moe_offload_cache.py:
66-292, tests/test_moe_offload_rebuild.py) with distinguishable banks: the
native LRU (ftm_lru_ensure / ftm_lru_materialize) must stage the same plan and
leave the same slot maps.  The byte copies themselves are GPU tests
(tests/test_gpu_offload.py)."""
import pytest
import torch

from ftmoe.moe.offload_cache import (_BANK_SCHEMAS, OffloadMoeCache, SlotWeightAccessor,
                                     gptq_int4_bytes_per_expert_slot)

L, E, S = 2, 4, 8
H, I = 16, 8


def _bank_values(layer, expert):
    base = 100 * (layer + 1) + 10 * (expert + 1)
    gate = torch.full((I, H), base + 0.0)
    up = torch.full((I, H), base + 1.0)
    down = torch.full((H, I), base + 2.0)
    return torch.cat([gate, up], dim=0), down


def _sources():
    return {
        "gate_up": [torch.stack([_bank_values(l, e)[0] for e in range(E)]) for l in range(L)],
        "down": [torch.stack([_bank_values(l, e)[1] for e in range(E)]) for l in range(L)],
    }


def _cache(slots):
    c = OffloadMoeCache(L, E, slots, "cpu", prefill_overlap=False)
    c.set_bank_sources(_sources())
    return c


def _assert_maps_consistent(c):
    for l in range(L):
        for e in range(E):
            s = int(c.slot_for_id[l, e])
            if s >= 0:
                assert int(c.id_of_slot[s]) == l * E + e


def test_prefill_materializes_whole_layer_identity_slots():
    c = _cache(S)
    c.materialize_layer(0)
    assert c.num_indices.item() == E
    assert [int(c.slot_for_id[0, e]) for e in range(E)] == list(range(E))
    assert c.evict_slots[:E].tolist() == list(range(E))
    assert c.src_indices[:E].tolist() == list(range(E))


def test_second_layer_evicts_first_layer_when_pool_holds_one():
    c = _cache(E)
    c.materialize_layer(0)
    c.materialize_layer(1)
    for e in range(E):
        assert int(c.slot_for_id[1, e]) != -1
        assert int(c.slot_for_id[0, e]) == -1
    assert c.resident_slots(1) == list(range(E))
    assert c.resident_slots(0) == []


def test_decode_hit_bumps_usage_and_stages_nothing():
    c = _cache(S)
    c.materialize_layer(0)
    c.materialize_layer(1)
    assert c.resident_slots(0) == [0, 1, 2, 3]
    assert c.resident_slots(1) == [4, 5, 6, 7]
    ids = torch.tensor([1], dtype=torch.int64)
    before = c.stat_missing.item()
    c.ensure_experts(1, ids)
    assert c.stat_missing.item() == before
    assert c.num_indices.item() == 0
    assert ids[0].item() == 1  # routing ids are never rewritten
    assert c.usage[int(c.slot_for_id[1, 1])].item() == c.step.item()


def test_decode_miss_takes_the_lru_slot():
    c = _cache(E)
    c.materialize_layer(0)
    c.step.fill_(3)
    c.usage[:] = torch.arange(E, dtype=torch.int64) + 1
    c.slot_for_id[0, 0] = -1  # as if evicted: routing expert 0 is a miss
    c.ensure_experts(0, torch.tensor([0], dtype=torch.int64))
    assert int(c.slot_for_id[0, 0]) == 0
    for e in range(1, E):
        assert int(c.slot_for_id[0, e]) == e
    assert c.num_indices.item() == 1
    assert c.evict_slots[0].item() == 0 and c.src_indices[0].item() == 0
    assert c.usage[0].item() == c.step.item()


def test_decode_miss_evicts_another_layers_lru_slot():
    c = _cache(E)
    for e in range(E):
        c.id_of_slot[e] = e
        c.slot_for_id[0, e] = e
    c.step.fill_(5)
    c.usage[:] = torch.arange(E, dtype=torch.int64) + 1
    c.ensure_experts(1, torch.tensor([0], dtype=torch.int64))
    assert int(c.slot_for_id[1, 0]) == 0
    assert int(c.slot_for_id[0, 0]) == -1
    assert int(c.slot_for_id[0, 1]) == 1
    assert int(c.slot_for_id[0, E - 1]) == E - 1
    assert c.num_indices.item() == 1


def test_misses_are_staged_in_ascending_expert_order_with_lru_victims():
    c = _cache(E)
    for e in range(E):  # layer 0 owns every slot; slot s last used at step 10 - s
        c.id_of_slot[e] = e
        c.slot_for_id[0, e] = e
    c.usage[:] = torch.tensor([10, 9, 8, 7], dtype=torch.int64)
    c.step.fill_(10)
    c.ensure_experts(1, torch.tensor([[3, 1], [1, 2]], dtype=torch.int64))
    n = c.num_indices.item()
    assert n == 3
    assert c.src_indices[:n].tolist() == [1, 2, 3]      # ascending expert id
    assert c.evict_slots[:n].tolist() == [3, 2, 1]      # oldest slot first
    assert c.stat_missing.item() == 3 and c.stat_calls.item() == 1
    _assert_maps_consistent(c)


def test_hit_miss_counters_and_reset_stats():
    c = _cache(S)
    c.materialize_layer(0)
    c.materialize_layer(1)
    base_missing, base_calls = c.stat_missing.item(), c.stat_calls.item()
    c.ensure_experts(1, torch.tensor([0], dtype=torch.int64))
    assert c.stat_calls.item() == base_calls + 1
    assert c.stat_missing.item() == base_missing
    assert c.decode_miss_stats() == {"missing": base_missing, "calls": base_calls + 1}
    c.reset_stats()
    assert c.stat_missing.item() == 0 and c.stat_calls.item() == 0


def test_bank_views_full_and_prefix():
    c = _cache(S)
    full = c.bank_views()
    assert len(full) == 2
    assert full[0].shape == (S, 2 * I, H) and full[1].shape == (S, H, I)
    assert c.bank_views(n=E)[0].shape == (E, 2 * I, H)


def test_cross_layer_eviction_keeps_slot_for_id_consistent():
    c = _cache(6)
    c.materialize_layer(0)
    c.materialize_layer(1)
    _assert_maps_consistent(c)
    assert int(c.slot_for_id[0, 0]) == -1
    assert int(c.slot_for_id[0, 1]) == -1
    for l in range(L):
        for e in range(E):
            c.ensure_experts(l, torch.tensor([e], dtype=torch.int64))
            _assert_maps_consistent(c)


def test_rebuild_resizes_pool_and_clears_state():
    c = _cache(S)
    c.materialize_layer(0)
    c.rebuild(6)
    assert c.cache_size == 6
    assert c.bank_views()[0].shape == (6, 2 * I, H)
    assert (c.slot_for_id == -1).all() and (c.id_of_slot == -1).all()
    assert c.step.item() == 0
    with pytest.raises(ValueError, match="must be >= num_experts"):
        c.rebuild(E - 1)


def test_constructor_and_wiring_errors():
    with pytest.raises(ValueError, match="unknown quant_format"):
        OffloadMoeCache(L, E, S, "cpu", quant_format="nope")
    with pytest.raises(ValueError, match="must be >= num_experts"):
        OffloadMoeCache(L, E, E - 1, "cpu")
    small = OffloadMoeCache(L, E, E - 1, "cpu", decode_only=True)  # a pool below one layer
    small.set_bank_sources(_sources())
    with pytest.raises(ValueError, match="cannot materialize a whole layer"):
        small.materialize_layer(0)
    small.ensure_experts(0, torch.tensor([0, 1, 2, 3]))
    assert small.num_indices.item() == 4 and sorted(small.evict_slots[:4].tolist()) == [0, 0, 1, 2]
    c = OffloadMoeCache(L, E, S, "cpu")
    with pytest.raises(ValueError, match="do not match"):
        c.set_bank_sources({"gate_up": _sources()["gate_up"]})
    with pytest.raises(AssertionError):
        c.bank_views()
    c.set_bank_sources(_sources())
    with pytest.raises(ValueError, match="Invalid materialize layer id"):
        c.materialize_layer(L)
    with pytest.raises(ValueError, match="expert ids"):
        c.ensure_experts(0, torch.tensor([E]))
    c.ensure_experts(0, torch.tensor([0]))
    with pytest.raises(RuntimeError, match="GPU slot pool"):
        c.copy_missing()


def test_bank_schemas_and_gptq_slot_bytes():
    assert _BANK_SCHEMAS["fp8_block"] == ("weight_gate_up", "scale_gate_up", "weight_down", "scale_down")
    assert set(_BANK_SCHEMAS) >= {"bf16", "gptq_int4", "fp8_block", "mxfp4", "int8_channel"}
    # C2 expert (H 2048, I 768, group 128): 2,451,456 bytes
    assert gptq_int4_bytes_per_expert_slot(2048, 768, 128) == 2_451_456
    with pytest.raises(ValueError):
        gptq_int4_bytes_per_expert_slot(0, 768, 128)


def test_accessor_refuses_to_guess():
    c = OffloadMoeCache(1, 2, 2, "cpu", quant_format="gptq_int4")
    c.set_bank_sources({b: [torch.zeros(2, 4, dtype=torch.int32)] for b in _BANK_SCHEMAS["gptq_int4"]})
    with pytest.raises(ValueError, match="gptq_group_size is not set"):
        SlotWeightAccessor(c, 8, torch.bfloat16)
    c8 = OffloadMoeCache(1, 2, 2, "cpu", quant_format="int8_channel")
    c8.set_bank_sources({b: [torch.zeros(2, 4, dtype=torch.int32)] for b in _BANK_SCHEMAS["int8_channel"]})
    with pytest.raises(ValueError, match="int8_k_gate_up / int8_k_down are not set"):
        SlotWeightAccessor(c8, 8, torch.bfloat16)
    cg = OffloadMoeCache(1, 2, 2, "cpu", quant_format="gguf_kquant")
    cg.set_bank_sources({b: [torch.zeros(2, 4, dtype=torch.uint8)] for b in _BANK_SCHEMAS["gguf_kquant"]})
    with pytest.raises(ValueError, match="no gfx950 kernel"):
        SlotWeightAccessor(cg, 8, torch.bfloat16)
    cf = OffloadMoeCache(1, 2, 2, "cpu", quant_format="fp8_block")
    cf.set_bank_sources({b: [torch.zeros(2, 4, dtype=torch.uint8)] for b in _BANK_SCHEMAS["fp8_block"]})
    acc = SlotWeightAccessor(cf, 8, torch.bfloat16)
    with pytest.raises(ValueError, match="get_gptq_packed is gptq_int4-only"):
        acc.get_gptq_packed(0)
    assert acc.get_fp8_packed(1)[4] == 128


# ---- the oracle's restatement of the LRU, and the native LRU against it

def test_oracle_lru_known_answers():
    """The reference's own cases (tests/test_moe_offload_cache.py:66-292, as
    restated above for the product) through the oracle's literal restatement."""
    import ftm_oracle as O

    st = O.lru_new(L, E, E)
    st.id_of_slot = list(range(E))
    O.lru_resync(st)
    st.usage, st.step = [10, 9, 8, 7], 10
    evict, src = O.lru_ensure(st, 1, [3, 1, 1, 2])
    assert src == [1, 2, 3] and evict == [3, 2, 1]
    assert st.missing == 3 and st.calls == 1
    st = O.lru_new(L, E, E)
    st.id_of_slot = list(range(E))
    O.lru_resync(st)
    st.usage, st.step = [1, 2, 3, 4], 5
    assert O.lru_ensure(st, 1, [0]) == ([0], [0])
    assert st.slot_for_id[E + 0] == 0 and st.slot_for_id[0] == -1 and st.slot_for_id[1] == 1
    # more misses than slots: once every slot carries this step, each further
    # miss takes min (step, slot) = slot 0, and the last one keeps it
    st = O.lru_new(1, 8, 3)
    evict, src = O.lru_ensure(st, 0, [5, 1, 7, 2, 6])
    assert src == [1, 2, 5, 6, 7] and evict == [0, 1, 2, 0, 0]
    assert st.id_of_slot == [7, 2, 5]


def _random_ids(rng, E, n):
    return rng.randint(0, E, size=n).tolist()


@pytest.mark.parametrize("Ln,En,Sn", [(3, 16, 5), (3, 16, 12), (2, 16, 40), (4, 8, 8)])
def test_native_lru_matches_oracle_on_random_sequences(Ln, En, Sn):
    import numpy as np

    import ftm_oracle as O

    rng = np.random.RandomState(Ln * 100 + En + Sn)
    c = OffloadMoeCache(Ln, En, Sn, "cpu", decode_only=Sn < En)
    st = O.lru_new(Ln, En, Sn)
    for call in range(60):
        layer = int(rng.randint(Ln))
        ids = _random_ids(rng, En, int(rng.randint(1, 2 * En)))
        c.ensure_experts(layer, torch.tensor(ids, dtype=torch.int64))
        evict, src = O.lru_ensure(st, layer, ids)
        n = int(c.num_indices.item())
        assert n == len(evict), call
        assert c.evict_slots[:n].tolist() == evict and c.src_indices[:n].tolist() == src, call
        assert c.slot_for_id.reshape(-1).tolist() == st.slot_for_id, call
        assert c.id_of_slot.tolist() == st.id_of_slot, call
        assert c.usage.tolist() == st.usage and int(c.step) == st.step, call
    assert c.decode_miss_stats() == {"missing": st.missing, "calls": st.calls}
