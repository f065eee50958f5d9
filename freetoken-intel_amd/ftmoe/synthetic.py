"""Seeded synthetic MoE layers for the benchmark configurations.

Each config follows the shapes and draw order of the measurement plan: one
``torch.Generator`` seeded with ``seed``, draws in the order
w13 -> w2 -> gate -> [shared expert w13, w2, gate] -> [router bias, expert
biases] -> x; weights N(0, 0.02), activations N(0, 1) rounded to bf16.  Weights
are quantized into the reference's bank layouts (python/freetoken/moe/
offload_cache.py:140-173) with :mod:`ftmoe.quant`.  There is no network access,
so every model here is random-init at the real architecture shape.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Optional

import torch

from . import quant


@dataclass(frozen=True)
class MoeConfig:
    name: str
    fmt: str
    E: int
    H: int
    I: int
    k: int
    T: int = 1
    shared_inter: int = 0
    group: int = 128            # fp8 block / gptq group
    int8_num_groups: int = 1    # 1 = per output channel
    route_mode: str = "softmax_topk"
    renormalize: bool = True
    act: str = "silu"
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0
    gate_bias: bool = False
    expert_bias: bool = False
    batches: tuple = (1,)
    prefill: Optional[int] = None
    bytes_per_expert: int = 0   # algorithmic bytes of one routed expert


CONFIGS = {
    # C1: INT8 per-output-channel, the reference's CPU-runnable case.
    "c1_int8": MoeConfig("c1_int8", "int8_channel", E=16, H=1024, I=512, k=2, T=4, batches=(4,),
                         bytes_per_expert=1_581_056),
    # C2: GPTQ int4 g128, 128 experts, top-8.
    "c2_gptq": MoeConfig("c2_gptq", "gptq_int4", E=128, H=2048, I=768, k=8, T=16, group=128,
                         batches=(1, 4, 16, 64), bytes_per_expert=2_451_456),
    # C3: FP8 128x128 block scales, 256 experts, top-8, shared bf16 expert (sigmoid gate).
    "c3_fp8": MoeConfig("c3_fp8", "fp8_block", E=256, H=2048, I=512, k=8, T=16, shared_inter=512,
                        batches=(1, 2, 4, 8, 16, 32, 64), prefill=2048, bytes_per_expert=3_146_496),
    # C4: MXFP4 e2m1/e8m0, 32 experts, top-4 on logits then softmax, clamped SwiGLU, biases.
    "c4_mxfp4": MoeConfig("c4_mxfp4", "mxfp4", E=32, H=2880, I=2880, k=4, T=32, group=32,
                          route_mode="topk_softmax", act="swiglu_oai", gate_bias=True, expert_bias=True,
                          batches=(1, 32, 128), prefill=4096, bytes_per_expert=13_236_480),
}

# Reduced shapes with the same structure, for oracle checks that must finish in seconds.
SMALL = {
    "c1_int8": replace(CONFIGS["c1_int8"], name="c1_small", E=8, H=256, I=128, k=2, T=5),
    "c2_gptq": replace(CONFIGS["c2_gptq"], name="c2_small", E=16, H=256, I=384, k=4, T=7),
    "c3_fp8": replace(CONFIGS["c3_fp8"], name="c3_small", E=32, H=256, I=256, k=4, T=6, shared_inter=128),
    "c4_mxfp4": replace(CONFIGS["c4_mxfp4"], name="c4_small", E=8, H=320, I=192, k=2, T=5),
}


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16)


def quantize_bank(fmt: str, w: torch.Tensor, which: str, *, group: int = 128, int8_num_groups: int = 1) -> dict:
    """Quantize stacked dense weights ``[E, N, K]`` (out, in) into the bank tensors
    of ``fmt`` for projection ``which`` (``"gate_up"`` / ``"down"``)."""
    if fmt == "bf16":
        return {which: _bf16(w)}
    if fmt == "fp8_block":
        q, s = quant.quantize_block_fp8(w, block=group)
        return {f"weight_{which}": q, f"scale_{which}": s}
    if fmt == "gptq_int4":
        qw, qz, sc = quant.quantize_gptq_int4(w.transpose(-1, -2), group_size=group)
        return {f"qweight_{which}": qw.contiguous(), f"qzeros_{which}": qz.contiguous(),
                f"scales_{which}": sc.contiguous()}
    if fmt == "int8_channel":
        E, N, K = w.shape
        gsz = K // int8_num_groups
        wg = w.reshape(E, N, int8_num_groups, gsz)
        codes, scale = quant.quantize_int8_channel(wg)  # per (row, group)
        return {f"weight_packed_{which}": quant.pack_int8_to_int32(codes.reshape(E, N, K)),
                f"weight_scale_{which}": scale.reshape(E, N, int8_num_groups).contiguous()}
    if fmt == "mxfp4":
        blocks, scales = quant.quantize_mxfp4_blocks(w)
        return {f"blocks_{which}": blocks, f"scales_{which}": scales}
    raise ValueError(f"unknown format {fmt!r}")


@dataclass
class SyntheticLayer:
    cfg: MoeConfig
    bank: dict                    # reference bank names -> [E, ...] tensors
    gate_w: torch.Tensor          # bf16 [E, H]
    x: torch.Tensor               # bf16 [T, H]
    gate_b: Optional[torch.Tensor] = None
    bias13: Optional[torch.Tensor] = None   # bf16 [E, 2I]
    bias2: Optional[torch.Tensor] = None    # bf16 [E, H]
    shared: Optional[dict] = None           # {"w13": [2Is, H], "w2": [H, Is], "gate": [1, H]} bf16
    extra: dict = field(default_factory=dict)

    def to(self, device) -> "SyntheticLayer":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return SyntheticLayer(self.cfg, {k: v.to(device) for k, v in self.bank.items()}, mv(self.gate_w),
                              mv(self.x), mv(self.gate_b), mv(self.bias13), mv(self.bias2),
                              {k: v.to(device) for k, v in self.shared.items()} if self.shared else None,
                              dict(self.extra))


def generate(cfg: MoeConfig, *, T: Optional[int] = None, seed: int = 0, device="cpu") -> SyntheticLayer:
    """Draw and quantize one layer of ``cfg`` (see module docstring for the order)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    T = cfg.T if T is None else T
    E, H, I = cfg.E, cfg.H, cfg.I

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)

    w13 = randn(E, 2 * I, H) * 0.02
    bank = quantize_bank(cfg.fmt, w13, "gate_up", group=cfg.group, int8_num_groups=cfg.int8_num_groups)
    del w13
    w2 = randn(E, H, I) * 0.02
    bank.update(quantize_bank(cfg.fmt, w2, "down", group=cfg.group, int8_num_groups=cfg.int8_num_groups))
    del w2
    gate_w = _bf16(randn(E, H) * 0.02)
    shared = None
    if cfg.shared_inter > 0:
        Is = cfg.shared_inter
        shared = {"w13": _bf16(randn(2 * Is, H) * 0.02), "w2": _bf16(randn(H, Is) * 0.02),
                  "gate": _bf16(randn(1, H) * 0.02)}
    gate_b = _bf16(randn(E) * 0.02) if cfg.gate_bias else None
    bias13 = _bf16(randn(E, 2 * I) * 0.02) if cfg.expert_bias else None
    bias2 = _bf16(randn(E, H) * 0.02) if cfg.expert_bias else None
    x = _bf16(randn(T, H))
    return SyntheticLayer(cfg, bank, gate_w, x, gate_b, bias13, bias2, shared)


def build_layer(syn: SyntheticLayer, *, slot_of_expert: Optional[torch.Tensor] = None, bank: Optional[dict] = None):
    """A :class:`~ftmoe.layer.MoeLayer` over ``syn`` (already on the GPU)."""
    from .banks import proj_from_bank
    from .layer import MoeLayer

    cfg = syn.cfg
    bank = syn.bank if bank is None else bank
    w13 = proj_from_bank(cfg.fmt, bank, which="gate_up", N=2 * cfg.I, K=cfg.H, group=cfg.group, bias=syn.bias13)
    w2 = proj_from_bank(cfg.fmt, bank, which="down", N=cfg.H, K=cfg.I, group=cfg.group, bias=syn.bias2)
    return MoeLayer(w13=w13, w2=w2, num_experts=cfg.E, hidden=cfg.H, inter=cfg.I, topk=cfg.k, gate_w=syn.gate_w,
                    gate_b=syn.gate_b, shared=syn.shared, route_mode=cfg.route_mode, renormalize=cfg.renormalize,
                    act=cfg.act, swiglu_alpha=cfg.swiglu_alpha, swiglu_limit=cfg.swiglu_limit,
                    slot_of_expert=slot_of_expert)


def algorithmic_bytes(cfg: MoeConfig, unique_experts: int, T: int) -> int:
    """B_alg of one layer forward: routed expert banks actually read + router
    weights + shared expert + activations in and out (bf16)."""
    b = unique_experts * cfg.bytes_per_expert + cfg.E * cfg.H * 2
    if cfg.shared_inter:
        b += 3 * cfg.H * cfg.shared_inter * 2 + cfg.H * 2
    if cfg.gate_bias:
        b += cfg.E * 2
    return b + 2 * T * cfg.H * 2
