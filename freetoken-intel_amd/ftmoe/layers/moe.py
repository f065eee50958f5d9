"""The reusable MoE layer the models build: the drop-in for the reference's
``Moe(nn.Module)`` (python/freetoken/layers/moe.py:29-83).

Same constructor (``hidden_size, num_experts, intermediate_size,
num_experts_per_tok, device, dtype, moe_backend, renormalize, activation,
apply_router_weight_on_input``), the same parameters for a loader to fill in
place (``gate`` an ``nn.Linear(hidden, E, bias=False)``; ``w1 [E, 2I, H]``
gate rows then up rows; ``w2 [E, H, I]``), and the same forward: router logits
of the flattened tokens, then the registered backend's
``forward(flat, w1, w2, gating, top_k, renormalize, activation,
apply_router_weight_on_input)``, output in the input's shape.

The router logits are this library's router kernel (the routing launch with
caller-visible logits), not a BLAS ``nn.Linear``: the same bf16 products,
summed in the kernel's fixed fp32 order and rounded to the activation dtype,
so the routing that the backend derives from them is reproducible bit for
bit.  Everything runs on the GPU; a CPU tensor raises.
"""
from __future__ import annotations

from typing import Optional, Union

import torch
import torch.nn as nn

from .. import _native as nat
from ..moe import create_moe_backend


class Moe(nn.Module):
    """Router (``gate``) + stacked expert banks (``w1``, ``w2``) + a routed-expert
    backend from the registry (``"fused"`` by default)."""

    def __init__(self, hidden_size: int, num_experts: int, intermediate_size: int, num_experts_per_tok: int,
                 device: Union[torch.device, str, None] = None, dtype: torch.dtype = torch.bfloat16,
                 moe_backend: str = "fused", renormalize: bool = True, activation: str = "silu",
                 apply_router_weight_on_input: bool = False) -> None:
        super().__init__()
        if isinstance(device, str):
            device = torch.device(device)
        self.hidden_size = int(hidden_size)
        self.num_experts = int(num_experts)
        self.intermediate_size = int(intermediate_size)
        self.top_k = int(num_experts_per_tok)
        self.renormalize = bool(renormalize)
        self.activation = activation
        self.apply_router_weight_on_input = bool(apply_router_weight_on_input)
        self.gate = nn.Linear(self.hidden_size, self.num_experts, bias=False, device=device, dtype=dtype)
        self.w1 = nn.Parameter(torch.empty(self.num_experts, 2 * self.intermediate_size, self.hidden_size,
                                           device=device, dtype=dtype))
        self.w2 = nn.Parameter(torch.empty(self.num_experts, self.hidden_size, self.intermediate_size,
                                           device=device, dtype=dtype))
        self.backend = create_moe_backend(moe_backend)
        self._router = None  # (key, MoeLayer) of the router launch over self.gate.weight

    def router_logits(self, flat: torch.Tensor) -> torch.Tensor:
        """``[T, E]`` router logits of ``flat [T, H]`` in ``flat``'s dtype."""
        from ..engine import _RouterOnly
        from ..layer import MoeLayer

        nat.require_gpu(flat, "hidden_states")
        gw = self.gate.weight
        nat.require_gpu(gw, "gate.weight")
        act_dtype = torch.bfloat16 if flat.dtype == torch.bfloat16 else torch.float32
        g = gw.detach()
        if g.dtype != torch.bfloat16:
            g = g.to(torch.bfloat16)
        g = g.contiguous()
        key = (g.data_ptr(), act_dtype, flat.device)
        if self._router is None or self._router[0] != key:
            layer = MoeLayer(w13=_RouterOnly.proj(g, self.hidden_size), w2=_RouterOnly.proj_down(g, self.hidden_size),
                             num_experts=self.num_experts, hidden=self.hidden_size, inter=_RouterOnly.I,
                             topk=min(self.top_k, self.num_experts), gate_w=g, route_mode="softmax_topk_lowp",
                             renormalize=self.renormalize, act_dtype=act_dtype)
            self._router = (key, layer, g)
        x = flat if flat.dtype == act_dtype else flat.to(act_dtype)
        _, _, logits = self._router[1].route(x.contiguous())
        return logits.to(flat.dtype)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        in_shape = hidden_states.shape
        flat = hidden_states.reshape(-1, in_shape[-1])
        gating = self.router_logits(flat)
        out = self.backend.forward(flat, self.w1, self.w2, gating, self.top_k, self.renormalize, self.activation,
                                   self.apply_router_weight_on_input)
        return out.view(in_shape)


__all__ = ["Moe"]
