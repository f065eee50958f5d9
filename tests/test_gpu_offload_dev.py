"""GPU: the slot pool's LRU and copy engine on the device (device_lru=True,
ftm_lru_ensure_dev / ftm_copy_slots_dev).

* after every call the device state (slot_for_id, id_of_slot, usage, step,
  the plan, the counters) equals the oracle's statement-by-statement
  restatement of ensure_experts (python/freetoken/moe/offload_cache.py:560-647),
  itself pinned to the reference's known answers on the CPU: pools smaller
  than a step's misses (every further miss through slot 0), pools of
  thousands of slots (the radix select over (usage, slot) keys), 512 experts,
  pairs without an expert (-1), several layers;
* chunk calls take the distinct experts' ranks [c * cap, (c + 1) * cap) and
  return the pairs outside the chunk as -1;
* the copy kernel moves exactly the staged rows of every bank (rows of
  several 64 KiB pieces, rows that are not a multiple of 16 bytes) and skips
  plan entries outside the banks;
* moe_offload_forward on the device path returns the host path's output
  bit for bit and leaves the same LRU state, chunked steps included."""
import ctypes

import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import assert_close, np_, oracle_spec, to_f32

from ftmoe import _native as nat
from ftmoe import synthetic as S
from ftmoe.moe.offload_cache import OffloadMoeCache, moe_offload_forward

pytestmark = pytest.mark.gpu


def _state_equal(c, st, plan, what):
    torch.cuda.synchronize()
    n = int(c._staged[0])
    if plan is None:
        assert n == 0, what
    else:
        evict, src = plan
        assert n == len(evict), what
        assert c.evict_slots[:n].tolist() == evict and c.src_indices[:n].tolist() == src, what
    assert c.slot_for_id.reshape(-1).tolist() == st.slot_for_id, what
    assert c.id_of_slot.tolist() == st.id_of_slot, what
    assert c.usage.tolist() == st.usage, what
    assert int(c.step) == st.step, what
    assert c.decode_miss_stats() == {"missing": st.missing, "calls": st.calls}, what


@pytest.mark.parametrize("Ln,En,Sn,calls", [(3, 16, 5, 40), (2, 64, 40, 40), (4, 256, 3000, 30), (2, 512, 64, 20),
                                            (3, 32, 1100, 30)])
def test_device_lru_matches_oracle(gpu, Ln, En, Sn, calls):
    rng = np.random.RandomState(Ln * 1000 + En + Sn)
    c = OffloadMoeCache(Ln, En, Sn, gpu, decode_only=Sn < En, device_lru=True)
    st = O.lru_new(Ln, En, Sn)
    for call in range(calls):
        layer = int(rng.randint(Ln))
        n = int(rng.randint(1, min(4 * En, 700)))
        ids = rng.randint(-1, En, size=n).astype(np.int32)  # -1: a pair without an expert
        print(f"device lru L={Ln} E={En} S={Sn} call {call} n={n}", flush=True)
        c.ensure_experts(layer, torch.from_numpy(ids).to(gpu))
        plan = O.lru_ensure(st, layer, [int(e) for e in ids if e >= 0])
        _state_equal(c, st, plan, f"call {call}")
    c.ensure_experts(0, torch.full((5,), -1, dtype=torch.int32, device=gpu))  # no expert: still a step
    _state_equal(c, st, O.lru_ensure(st, 0, []), "empty call")
    c.check_status()


def test_device_lru_flags_out_of_range_ids(gpu):
    c = OffloadMoeCache(1, 8, 8, gpu, device_lru=True)
    c.ensure_experts(0, torch.tensor([1, 9, 2], device=gpu))
    with pytest.raises(ValueError, match="must lie in"):
        c.check_status()
    # the valid ids were ensured, the bad one ignored
    torch.cuda.synchronize()
    assert int(c._staged[0]) == 2 and c.src_indices[:2].tolist() == [1, 2]
    c.check_status()  # cleared


@pytest.mark.parametrize("cap", [3, 7, 64])
def test_device_lru_chunks_match_oracle(gpu, cap):
    rng = np.random.RandomState(cap)
    Ln, En, Sn = 2, 32, 9
    c = OffloadMoeCache(Ln, En, Sn, gpu, decode_only=True, device_lru=True)
    st = O.lru_new(Ln, En, Sn)
    for step in range(8):
        layer = step % Ln
        ids = rng.randint(-1, En, size=(6, 4)).astype(np.int32)
        ids_dev = torch.from_numpy(ids).to(gpu)
        for ch in range(-(-min(ids.size, En) // cap)):
            ids_c = c.ensure_experts_chunk(layer, ids_dev, ch, cap, want_ids=True)
            plan, members = O.lru_ensure_chunk(st, layer, ids.reshape(-1).tolist(), ch, cap)
            want = np.where(np.isin(ids, members), ids, -1)
            assert ids_c.shape == ids_dev.shape and ids_c.cpu().numpy().tolist() == want.tolist(), (step, ch)
            _state_equal(c, st, plan, f"step {step} chunk {ch}")


def _pinned(t):
    return t.contiguous().pin_memory()


def test_copy_kernel_moves_staged_rows(gpu):
    rng = np.random.RandomState(3)
    rows, slots = 6, 5
    big = _pinned(torch.from_numpy(rng.randint(0, 256, size=(rows, 200_000), dtype=np.uint8)))  # 4 pieces
    odd = _pinned(torch.from_numpy(rng.randint(0, 256, size=(rows, 37), dtype=np.uint8)))  # byte path
    dev_big = torch.zeros((slots, 200_000), dtype=torch.uint8, device=gpu)
    dev_odd = torch.zeros((slots, 37), dtype=torch.uint8, device=gpu)
    evict = torch.tensor([4, 0, 2, 3, 1], dtype=torch.int32, device=gpu)
    src = torch.tensor([5, 1, 3, 99, 0], dtype=torch.int32, device=gpu)  # row 99: outside the bank, skipped
    num = torch.tensor([4], dtype=torch.int32, device=gpu)  # the fifth entry is past num_staged
    descs = (nat.FtmBankCopy * 2)(nat.FtmBankCopy(big.data_ptr(), dev_big.data_ptr(), 200_000),
                                  nat.FtmBankCopy(odd.data_ptr(), dev_odd.data_ptr(), 37))
    rc = nat.lib().ftm_copy_slots_dev(descs, 2, rows, slots, evict.data_ptr(), src.data_ptr(), num.data_ptr(), 5,
                                      torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == nat.OK
    torch.cuda.synchronize()
    for slot, row in ((4, 5), (0, 1), (2, 3)):
        assert torch.equal(dev_big[slot].cpu(), big[row]), slot
        assert torch.equal(dev_odd[slot].cpu(), odd[row]), slot
    for slot in (3, 1):  # skipped entry, entry past the count: untouched
        assert int(dev_big[slot].abs().sum()) == 0 and int(dev_odd[slot].abs().sum()) == 0
    # a device pointer is not pinned host memory: refused before any launch
    # (host_rows = 1 skips every entry of this plan even if it were not)
    bad = (nat.FtmBankCopy * 1)(nat.FtmBankCopy(dev_odd.data_ptr(), dev_big.data_ptr(), 37))
    assert nat.lib().ftm_copy_slots_dev(bad, 1, 1, slots, evict.data_ptr(), src.data_ptr(), num.data_ptr(), 5,
                                        torch.cuda.current_stream(gpu).cuda_stream) == nat.ERR_HIP


def _bank_values(layer, expert, I=8, H=16):
    base = 100 * (layer + 1) + 10 * (expert + 1)
    gate_up = torch.cat([torch.full((I, H), base + 0.0), torch.full((I, H), base + 1.0)])
    return gate_up, torch.full((H, I), base + 2.0)


def test_device_copy_missing_streams_the_staged_rows(gpu):
    Ln, En = 2, 4
    c = OffloadMoeCache(Ln, En, 3, gpu, decode_only=True, device_lru=True)
    c.set_bank_sources({"gate_up": [torch.stack([_bank_values(l, e)[0] for e in range(En)]) for l in range(Ln)],
                        "down": [torch.stack([_bank_values(l, e)[1] for e in range(En)]) for l in range(Ln)]})
    for layer, ids in ((0, [2, 0]), (1, [3]), (0, [1, 2])):
        c.ensure_experts(layer, torch.tensor(ids, device=gpu))
        c.copy_missing()
        torch.cuda.synchronize()
        for s, fid in enumerate(c.id_of_slot.tolist()):
            if fid >= 0:
                gu, dn = _bank_values(fid // En, fid % En)
                assert torch.equal(c.bank_caches["gate_up"][s].cpu(), gu), (layer, s)
                assert torch.equal(c.bank_caches["down"][s].cpu(), dn), (layer, s)
        sl = c.slot_of_expert(layer)
        assert sl.is_cuda and all(sl[e].item() >= 0 for e in ids)


def _fp8_pools(gpu, slots, seeds=(31, 32)):
    cfg = S.SMALL["c3_fp8"]
    syns = [S.generate(cfg, T=12, seed=s) for s in seeds]
    caches = []
    for dev_lru in (False, True):
        c = OffloadMoeCache(len(syns), cfg.E, slots, gpu, quant_format="fp8_block", decode_only=slots < cfg.E,
                            device_lru=dev_lru)
        c.set_bank_sources({b: [syn.bank[b] for syn in syns] for b in c.bank_schema})
        caches.append(c)
    return cfg, syns, caches


@pytest.mark.parametrize("slots", [6, 24])
def test_device_offload_forward_matches_host_path(gpu, slots):
    cfg, syns, (ch, cd) = _fp8_pools(gpu, slots)
    rng = np.random.RandomState(11 + slots)
    T = 5
    for step in range(6):
        layer_id = step % 2
        syn = syns[layer_id]
        x = syn.x[:T].to(gpu)
        ids = np.stack([rng.choice(cfg.E, cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
        w = O.round_bf16(rng.rand(T, cfg.k).astype(np.float32))
        ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
        shared = {k: v.to(gpu) for k, v in syn.shared.items()}
        print(f"offload forward slots={slots} step {step} distinct={len(np.unique(ids))}", flush=True)
        out_h = moe_offload_forward(x, ids_d, w_d, ch, layer_id, intermediate=cfg.I, shared=shared)
        out_d = moe_offload_forward(x, ids_d, w_d, cd, layer_id, intermediate=cfg.I, shared=shared)
        torch.cuda.synchronize()
        assert torch.equal(out_d, out_h), step
        ref = O.layer_reference(oracle_spec(syn), np_(syn.x[:T]), ids=ids, w=w)
        assert_close(to_f32(out_d), ref["out"], what=f"device pool step {step}")
        assert cd.slot_for_id.cpu().tolist() == ch.slot_for_id.tolist(), step
        assert cd.id_of_slot.cpu().tolist() == ch.id_of_slot.tolist(), step
        assert cd.usage.cpu().tolist() == ch.usage.tolist() and int(cd.step) == int(ch.step), step
    assert cd.decode_miss_stats() == ch.decode_miss_stats()
    cd.check_status()


def test_copy_kernel_applies_repeated_slots_in_plan_order(gpu):
    """A plan that names one slot more than once (ensure_experts passes every
    miss beyond the unstamped slots through slot 0) lands the last such row,
    as copy_missing's in-order copies do (offload_cache.py:651-674)."""
    rows, slots = 6, 4
    bank = _pinned(torch.arange(rows, dtype=torch.uint8)[:, None].repeat(1, 70_000) + 1)  # row r holds r + 1
    pool = torch.zeros((slots, 70_000), dtype=torch.uint8, device=gpu)
    evict = torch.tensor([3, 0, 0, 0], dtype=torch.int32, device=gpu)
    src = torch.tensor([5, 1, 2, 4], dtype=torch.int32, device=gpu)
    num = torch.tensor([4], dtype=torch.int32, device=gpu)
    descs = (nat.FtmBankCopy * 1)(nat.FtmBankCopy(bank.data_ptr(), pool.data_ptr(), 70_000))
    assert nat.lib().ftm_copy_slots_dev(descs, 1, rows, slots, evict.data_ptr(), src.data_ptr(), num.data_ptr(), 4,
                                        torch.cuda.current_stream(gpu).cuda_stream) == nat.OK
    torch.cuda.synchronize()
    assert torch.equal(pool[3].cpu(), bank[5]) and torch.equal(pool[0].cpu(), bank[4])
    assert int(pool[1].sum()) == 0 and int(pool[2].sum()) == 0


def test_device_pool_smaller_than_the_step_keeps_the_last_miss(gpu):
    """ensure_experts on a pool smaller than the step's distinct experts (the
    misses beyond the pool pass through slot 0, the last one stays): after
    copy_missing every slot holds exactly the bank row its id_of_slot names,
    on the device path as on the host path."""
    Ln, En, Sn = 1, 8, 3
    srcs = {"gate_up": [torch.stack([_bank_values(0, e)[0] for e in range(En)])],
            "down": [torch.stack([_bank_values(0, e)[1] for e in range(En)])]}
    for dev_lru in (True, False):
        c = OffloadMoeCache(Ln, En, Sn, gpu, decode_only=True, device_lru=dev_lru)
        c.set_bank_sources(srcs)
        for ids in ([0, 1, 2, 3, 4, 5], [6, 7, 1], [2, 3, 4, 5, 6, 7, 0]):
            c.ensure_experts(0, torch.tensor(ids, device=gpu))
            c.copy_missing()
            torch.cuda.synchronize()
            for s, fid in enumerate(c.id_of_slot.tolist()):
                assert fid >= 0
                gu, dn = _bank_values(0, fid % En)
                assert torch.equal(c.bank_caches["gate_up"][s].cpu(), gu), (dev_lru, ids, s, fid)
                assert torch.equal(c.bank_caches["down"][s].cpu(), dn), (dev_lru, ids, s, fid)
