"""Adapters between the product's torch banks and the oracle's numpy banks,
plus the output tolerance of the parity contract."""
from __future__ import annotations

import numpy as np
import torch

import ftm_oracle as O

# bf16 outputs vs the fp32-accumulated oracle: |got - ref| <= ATOL + RTOL * |ref|
ATOL = 2e-2
RTOL = 1e-2


def np_(t):
    if t is None:
        return None
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def oracle_proj(fmt, bank, which, N, K, group, bias=None):
    b = np_(bias)
    if fmt == "bf16":
        return O.OracleProj("bf16", np_(bank[which]), N, K, bias=b)
    if fmt == "fp8_block":
        return O.OracleProj(fmt, np_(bank[f"weight_{which}"]), N, K, s=np_(bank[f"scale_{which}"]), group=group, bias=b)
    if fmt == "gptq_int4":
        return O.OracleProj(fmt, np_(bank[f"qweight_{which}"]), N, K, s=np_(bank[f"scales_{which}"]),
                            z=np_(bank[f"qzeros_{which}"]), group=group, bias=b)
    if fmt == "int8_channel":
        s = np_(bank[f"weight_scale_{which}"])
        return O.OracleProj(fmt, np_(bank[f"weight_packed_{which}"]), N, K, s=s, group=K // s.shape[-1], bias=b)
    if fmt == "mxfp4":
        return O.OracleProj(fmt, np_(bank[f"blocks_{which}"]), N, K, s=np_(bank[f"scales_{which}"]), group=32, bias=b)
    raise ValueError(fmt)


def oracle_spec(syn) -> dict:
    c = syn.cfg
    spec = dict(fmt=c.fmt, E=c.E, H=c.H, I=c.I, k=c.k, route_mode=c.route_mode, renormalize=c.renormalize,
                act=c.act, alpha=c.swiglu_alpha, limit=c.swiglu_limit,
                w13=oracle_proj(c.fmt, syn.bank, "gate_up", 2 * c.I, c.H, c.group, syn.bias13),
                w2=oracle_proj(c.fmt, syn.bank, "down", c.H, c.I, c.group, syn.bias2),
                gate_w=np_(syn.gate_w), gate_b=np_(syn.gate_b))
    if syn.shared is not None:
        spec["shared"] = {k: np_(v) for k, v in syn.shared.items()}
    return spec


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what="output"):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} elements out of tolerance "
                             f"(atol {atol}, rtol {rtol}); worst at {i}: got {got[i]}, ref {ref[i]}")


def to_f32(t):
    return t.detach().float().cpu().numpy()


# Relative RMS error bound of the MXFP4 decode path (activations as two e4m3
# terms): a bf16 output and a bf16 intermediate keep ||got - ref|| / ||ref||
# near 2e-3; the input rounded to one e4m3 term (the lo term lost) puts it
# near 3e-2 (the oracle-side check in test_mx_quant.py).
MX_REL_RMS = 8e-3


def rel_rms(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def wide_range_x(T, H, seed):
    """bf16 [T, H] inputs whose elements span 2^-14 .. 2^3 inside each 32-wide block."""
    g = torch.Generator().manual_seed(seed)
    e = torch.randint(-14, 3, (T, H), generator=g).float()
    return (torch.randn(T, H, generator=g) * torch.exp2(e)).to(torch.bfloat16)
