"""The reference's caller-side classes as drop-ins, on the CPU:
``CpuMoeExecutor`` (python/freetoken/moe/cpu_executor.py:51-144) against the
oracle's expert layer with fp32 ``h`` (the reference CPU kernel's
arithmetic) and against the reference's own CPU kernel where it is built;
``Moe`` (python/freetoken/layers/moe.py:29-83): the reference's constructor,
parameter shapes and registry backend, and no CPU fallback."""
import numpy as np
import pytest
import torch

import ftm_oracle as O

from ftmoe.layers import Moe
from ftmoe.moe.cpu_executor import CpuMoeExecutor


def _banks(E, H, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    dn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    return gu, dn


def _routing(T, E, k, seed):
    rng = np.random.RandomState(seed)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.rand(T, k).astype(np.float32)
    return torch.from_numpy(ids), torch.from_numpy(w / w.sum(1, keepdims=True))


def _oracle(flat, ids, w, gu, dn):
    E, I2, H = gu.shape
    fmt = "bf16" if gu.dtype == torch.bfloat16 else "fp32"
    a = gu.contiguous().view(torch.int16).numpy().view(np.uint16) if fmt == "bf16" else gu.float().numpy()
    b = dn.contiguous().view(torch.int16).numpy().view(np.uint16) if fmt == "bf16" else dn.float().numpy()
    p13, p2 = O.OracleProj(fmt, np.ascontiguousarray(a), I2, H), O.OracleProj(fmt, np.ascontiguousarray(b), H, I2 // 2)
    return O.moe_experts(p13, p2, flat.float().numpy(), ids.numpy().astype(np.int32), w.numpy(), E=E,
                         h_bf16=False, x_bf16=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("threads", [0, 1, 3])
def test_cpu_executor_matches_oracle(dtype, threads):
    E, H, I, T, k = 8, 128, 64, 5, 2
    gu, dn = _banks(E, H, I, dtype, 1)
    ids, w = _routing(T, E, k, 2)
    flat = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(dtype)
    ex = CpuMoeExecutor(E, I, threads=threads)
    got = ex.forward(flat, ids, w, gu, dn)
    assert got.dtype == flat.dtype and got.shape == flat.shape and got.device == flat.device
    ref = _oracle(flat, ids, w, gu, dn)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    np.testing.assert_allclose(got.float().numpy(), ref, rtol=tol, atol=tol * np.abs(ref).max())
    again = ex(flat, ids, w, gu, dn)  # cached descriptor, same result
    assert torch.equal(again, got)


def test_cpu_executor_empty_batch_and_errors():
    E, H, I = 4, 64, 32
    gu, dn = _banks(E, H, I, torch.float32, 4)
    ex = CpuMoeExecutor(E, I)
    out = ex.forward(torch.zeros(0, H), torch.zeros(0, 2, dtype=torch.int64), torch.zeros(0, 2), gu, dn)
    assert out.shape == (0, H)
    with pytest.raises(ValueError, match="do not match"):
        CpuMoeExecutor(E + 1, I).forward(torch.zeros(1, H), torch.zeros(1, 2, dtype=torch.int64), torch.ones(1, 2),
                                         gu, dn)
    with pytest.raises(ValueError, match="one \\[T, H\\] batch"):
        ex.forward(torch.zeros(2, H), torch.zeros(3, 2, dtype=torch.int64), torch.ones(3, 2), gu, dn)


@pytest.mark.skipif(not O.ref_cpu_moe_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_cpu_executor_matches_reference_cpu_kernel():
    """The reference's own freetoken_cpu_moe_forward_fast on the same fp32 banks."""
    E, H, I, T, k = 6, 96, 48, 4, 2
    gu, dn = _banks(E, H, I, torch.float32, 5)
    ids, w = _routing(T, E, k, 6)
    flat = torch.randn(T, H, generator=torch.Generator().manual_seed(7))
    got = CpuMoeExecutor(E, I, threads=1).forward(flat, ids, w, gu, dn)
    ref = O.ref_cpu_moe_forward_fast(flat.numpy(), ids.numpy().astype(np.int32), w.numpy(), gu.numpy(), dn.numpy(),
                                     threads=1)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-4, atol=1e-5)


def test_moe_module_has_the_reference_layout_and_no_cpu_fallback():
    m = Moe(64, 8, 32, 2, device="cpu")
    assert isinstance(m.gate, torch.nn.Linear) and m.gate.weight.shape == (8, 64) and m.gate.bias is None
    assert m.w1.shape == (8, 64, 64) and m.w2.shape == (8, 64, 32)
    assert {n for n, _ in m.named_parameters()} == {"gate.weight", "w1", "w2"}
    assert m.top_k == 2 and m.renormalize and m.activation == "silu" and not m.apply_router_weight_on_input
    with pytest.raises(KeyError, match="not registered"):
        Moe(64, 8, 32, 2, device="cpu", moe_backend="nope")
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        m(torch.zeros(3, 64, dtype=torch.bfloat16))


def test_registry_has_the_reference_keys():
    """python/freetoken/moe/__init__.py:142-167: fused, offload, cpu, hybrid; the
    three engine-selection hooks raise from the dense forward, naming the
    entry point a block calls instead."""
    from ftmoe.moe import SUPPORTED_MOE_BACKENDS, create_moe_backend

    assert set(SUPPORTED_MOE_BACKENDS) == {"fused", "offload", "cpu", "hybrid"}
    for key, entry in (("offload", "moe_offload_forward"), ("cpu", "CpuMoeExecutor"), ("hybrid", "moe_hybrid_forward")):
        b = create_moe_backend(key)
        with pytest.raises(NotImplementedError, match=entry):
            b.forward(None, None, None, None, 2, True, "silu", False)
