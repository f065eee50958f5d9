"""Router top-k + grouped SwiGLU expert GEMM + weighted combine on dense banks
(python/freetoken/kernel/triton/fused_moe.py:64-161), as gfx950 HIP kernels.

Softmax stays in the gating dtype before top-k (fused_moe.py:92-93), ties go
to the lower expert id, the optional renorm divides in that dtype, and the
router weights are rounded to the activation dtype (:96).  Experts are
grouped on the device (counting sort, no host sync), each expert's weights are
read once per step, and the k contributions of a token are summed in fixed
slot order in fp32 (no atomics)."""
from __future__ import annotations

import torch

from .. import _native as nat
from ..banks import Proj
from ..layer import ACTIVATIONS, MoeLayer


def fused_moe(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    gating: torch.Tensor,
    topk: int,
    renormalize: bool,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
) -> torch.Tensor:
    """``hidden_states [T, H]``, ``w1 [E, 2I, H]`` (gate||up), ``w2 [E, H, I]``,
    ``gating [T, E]`` router logits -> ``[T, H]``."""
    if gating.shape[0] != hidden_states.shape[0]:
        raise ValueError(f"gating rows ({gating.shape[0]}) != hidden_states rows ({hidden_states.shape[0]})")
    if activation not in ACTIVATIONS or activation == "swiglu_oai":
        raise ValueError(f"unsupported MoE activation: {activation!r}")
    for name, t in (("hidden_states", hidden_states), ("w1", w1), ("w2", w2), ("gating", gating)):
        nat.require_gpu(t, name)
    T, H = hidden_states.shape
    E, I2, _ = w1.shape
    I = I2 // 2
    out_dtype = hidden_states.dtype
    act_dtype = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
    wdt = w1.dtype
    if wdt == torch.bfloat16:
        fmt, w1c, w2c = "bf16", w1.contiguous(), w2.contiguous()
    else:
        fmt, w1c, w2c = "fp32", w1.to(torch.float32).contiguous(), w2.to(torch.float32).contiguous()
    layer = MoeLayer(w13=Proj(fmt, w1c, 2 * I, H), w2=Proj(fmt, w2c, H, I), num_experts=E, hidden=H, inter=I,
                     topk=topk, route_mode="softmax_topk_lowp", renormalize=renormalize, act=activation,
                     apply_router_weight_on_input=apply_router_weight_on_input, act_dtype=act_dtype)
    ids, w, _ = layer.route(logits=gating)
    out = layer.forward_routed(hidden_states.to(act_dtype), ids, w)
    return out if out.dtype == out_dtype else out.to(out_dtype)
