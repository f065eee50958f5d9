"""The host-CPU expert kernel of the hybrid split (ftm_cpu_moe_forward,
csrc/ftm_cpu.cpp) on the CPU: every bank format against the oracle (fp32 h,
as the reference CPU backend computes it), the AVX-512 and scalar paths, one
and several threads, expert masks, the async submit/wait worker and its
errors, and the split rule of the reference's hybrid forward."""
from dataclasses import replace

import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import np_, oracle_spec

from ftmoe import _native as nat
from ftmoe import synthetic as S
from ftmoe.moe import hybrid as HY

NAMES = ["c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"]


def _host(syn):
    c = syn.cfg
    int8_k = (c.H, c.I) if c.fmt == "int8_channel" else None
    return HY.host_layer_from_bank(c.fmt, syn.bank, num_experts=c.E, intermediate=c.I, topk=c.k, group=c.group,
                                   int8_k=int8_k, bias13=syn.bias13, bias2=syn.bias2, act=c.act)


def _routing(syn, T, seed):
    rng = np.random.RandomState(seed)
    ids = np.stack([rng.choice(syn.cfg.E, syn.cfg.k, replace=False) for _ in range(T)]).astype(np.int32)
    return ids, rng.rand(T, syn.cfg.k).astype(np.float32)


def _ref(syn, x, ids, w, mask=None):
    spec = oracle_spec(syn)
    if mask is not None:
        w = np.where(mask[ids] != 0, w, 0.0).astype(np.float32)
    return O.moe_experts(spec["w13"], spec["w2"], x, ids, w, E=syn.cfg.E, act=syn.cfg.act, alpha=syn.cfg.swiglu_alpha,
                         limit=syn.cfg.swiglu_limit, h_bf16=False, x_bf16=False)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("force_scalar", [False, True])
def test_cpu_half_matches_oracle(name, force_scalar):
    cfg = replace(S.SMALL[name], E=6)
    syn = S.generate(cfg, T=5, seed=500)
    L, keep = _host(syn)
    x = syn.x.float()
    ids, w = _routing(syn, 5, 1)
    got = HY.cpu_moe_forward(L, x, torch.from_numpy(ids), torch.from_numpy(w), force_scalar=force_scalar)
    ref = _ref(syn, x.numpy(), ids, w)
    np.testing.assert_allclose(got.numpy(), ref, rtol=2e-4, atol=2e-5 * np.abs(ref).max())


def test_avx512_path_equals_scalar_path_closely_and_threads_agree():
    syn = S.generate(replace(S.SMALL["c3_fp8"], E=8), T=9, seed=501)
    L, keep = _host(syn)
    x = syn.x.float()
    ids, w = _routing(syn, 9, 2)
    ids_t, w_t = torch.from_numpy(ids), torch.from_numpy(w)
    a = HY.cpu_moe_forward(L, x, ids_t, w_t, threads=1)
    b = HY.cpu_moe_forward(L, x, ids_t, w_t, threads=1, force_scalar=True)
    c = HY.cpu_moe_forward(L, x, ids_t, w_t, threads=3)
    np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(a.numpy(), c.numpy(), rtol=1e-5, atol=1e-6)
    assert torch.equal(c, HY.cpu_moe_forward(L, x, ids_t, w_t, threads=3))  # deterministic per thread count


def test_expert_mask_and_async_worker():
    syn = S.generate(replace(S.SMALL["c2_gptq"], E=8), T=6, seed=502)
    L, keep = _host(syn)
    x = syn.x.float().contiguous()
    ids, w = _routing(syn, 6, 3)
    mask = np.zeros(8, np.uint8)
    mask[[1, 4, 5]] = 1
    got = HY.cpu_moe_forward(L, x, torch.from_numpy(ids), torch.from_numpy(w), torch.from_numpy(mask))
    ref = _ref(syn, x.numpy(), ids, w, mask)
    np.testing.assert_allclose(got.numpy(), ref, rtol=2e-4, atol=2e-5 * np.abs(ref).max())
    out = torch.empty_like(x)
    job = HY.CpuJob(L, x, torch.from_numpy(ids), torch.from_numpy(w), torch.from_numpy(mask), out, keep)
    assert torch.equal(job.result(), got)
    with pytest.raises(RuntimeError, match="twice"):
        job.result()
    assert nat.lib().ftm_cpu_moe_wait(12345) == nat.ERR_HANDLE


def test_cpu_half_argument_errors():
    syn = S.generate(replace(S.SMALL["c3_fp8"], E=4), T=2, seed=503)
    L, keep = _host(syn)
    x = torch.zeros(2, syn.cfg.H)
    ids = torch.tensor([[0, 9, 1, 2], [0, 1, 2, 3]], dtype=torch.int32)[:, :syn.cfg.k]
    w = torch.ones(2, syn.cfg.k)
    with pytest.raises(nat.FtmError, match="code -2"):
        HY.cpu_moe_forward(L, x, ids, w)  # an id >= E
    assert nat.lib().ftm_cpu_moe_forward(None, None, 0, None, None, None, 0, 0, None) == nat.ERR_NULL


def test_split_rule_matches_the_reference():
    """qwen3_moe/__init__.py:733-752: n distinct experts, n_fetch = round(n f)
    clamped to [1, n - 1] and max_fetch, the CPU takes the lowest ids."""
    ids = torch.tensor([[7, 3, 9], [3, 1, 12]])
    assert HY.split_experts(ids, 0.5) == {1, 3, 7}       # n = 5: round(2.5) = 2 fetched (half to even), 3 on the CPU
    assert HY.split_experts(ids, 0.3) == {1, 3, 7}       # round(1.5) = 2 fetched
    assert HY.split_experts(ids, 0.99) == {1}            # n_fetch clamped to n - 1
    assert HY.split_experts(ids, 0.01) == {1, 3, 7, 9}   # at least one fetched
    assert HY.split_experts(ids, 0.8, max_fetch=1) == {1, 3, 7, 9}
    assert HY.split_experts(ids, 1.0) is None and HY.split_experts(ids, 0.0) is None
    assert HY.split_experts(torch.tensor([[4, -1]]), 0.5) is None  # one expert: nothing to split


@pytest.mark.skipif(not O.ref_cpu_moe_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("name", ["c1_int8", "c2_gptq", "c3_fp8"])
def test_cpu_half_matches_the_reference_cpu_kernel(name):
    """Against the reference's own CPU MoE (cpu_moe.cpp freetoken_cpu_moe_forward_fast,
    built unmodified into oracle/_ref) on the same experts dequantized to fp32 (the
    reference's CPU path takes dense fp32 banks: python/freetoken/kernel/cpu_moe.py:
    460-461): the packed-bank decode and the fp32 SwiGLU + combine agree to fp32
    reassociation."""
    cfg = replace(S.SMALL[name], E=6)
    syn = S.generate(cfg, T=5, seed=504)
    L, keep = _host(syn)
    spec = oracle_spec(syn)
    gu = np.stack([O.dequant(spec["w13"], e) for e in range(cfg.E)]).astype(np.float32)
    dn = np.stack([O.dequant(spec["w2"], e) for e in range(cfg.E)]).astype(np.float32)
    x = syn.x.float()
    ids, w = _routing(syn, 5, 4)
    got = HY.cpu_moe_forward(L, x, torch.from_numpy(ids), torch.from_numpy(w), threads=2)
    ref = O.ref_cpu_moe_forward_fast(x.numpy(), ids, w, gu, dn, threads=1)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


def test_hybrid_step_with_a_failing_gpu_half_frees_the_worker(monkeypatch):
    """A GPU half that raises (bad ids, a stale slot, a pool-size error) must
    not leave the CPU job running on freed buffers or holding the worker's
    only slot: the error propagates, and the next hybrid step completes."""
    from ftmoe.moe import offload_cache as OC

    cfg = replace(S.SMALL["c3_fp8"], E=8)
    syn = S.generate(cfg, T=4, seed=504)
    cache = OC.OffloadMoeCache(1, cfg.E, cfg.E, "cpu", quant_format="fp8_block")
    cache.set_bank_sources({b: [syn.bank[b]] for b in OC._BANK_SCHEMAS["fp8_block"]})
    ids, w = _routing(syn, 4, 5)
    ids_t, w_t = torch.from_numpy(ids), torch.from_numpy(w)
    calls = []

    def failing_gpu_half(*a, **kw):
        calls.append(1)
        raise IndexError("stale slot map (simulated)")

    monkeypatch.setattr(OC, "moe_offload_forward", failing_gpu_half)
    for _ in range(2):  # a second failing step: the worker's slot was freed by the first
        with pytest.raises(IndexError, match="simulated"):
            HY.moe_hybrid_forward(syn.x, ids_t, w_t, cache, 0, intermediate=cfg.I, fetch_fraction=0.5)
    assert len(calls) == 2

    def cpu_only_gpu_half(flat, ids_gpu, top_w, cache_, layer_id, **kw):
        return torch.zeros(flat.shape, dtype=flat.dtype)

    monkeypatch.setattr(OC, "moe_offload_forward", cpu_only_gpu_half)
    got = HY.moe_hybrid_forward(syn.x, ids_t, w_t, cache, 0, intermediate=cfg.I, fetch_fraction=0.5)
    mask = np.zeros(cfg.E, np.uint8)
    mask[sorted(HY.split_experts(ids_t, 0.5))] = 1
    L, keep = _host(syn)
    want = HY.cpu_moe_forward(L, syn.x.float(), ids_t, w_t, torch.from_numpy(mask)).to(syn.x.dtype)
    assert torch.equal(got, want)


def test_uncollected_cpu_job_is_waited_for_on_collection():
    """A CpuJob dropped without result() is waited for when collected, so the
    next submit does not block on the worker's only slot."""
    import gc

    syn = S.generate(replace(S.SMALL["c3_fp8"], E=6), T=3, seed=505)
    L, keep = _host(syn)
    x = syn.x.float().contiguous()
    ids, w = _routing(syn, 3, 6)
    job = HY.CpuJob(L, x, torch.from_numpy(ids), torch.from_numpy(w), None, torch.empty_like(x), keep)
    del job
    gc.collect()
    job2 = HY.CpuJob(L, x, torch.from_numpy(ids), torch.from_numpy(w), None, torch.empty_like(x), keep)
    assert torch.equal(job2.result(), HY.cpu_moe_forward(L, x, torch.from_numpy(ids), torch.from_numpy(w)))
