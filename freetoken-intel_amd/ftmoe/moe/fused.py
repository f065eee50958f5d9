"""The ``fused`` MoE backend (python/freetoken/moe/fused.py:19-50): experts
resident in HBM, routed and computed by the gfx950 HIP kernels."""
from __future__ import annotations

import torch

from ..kernel.moe_impl import fused_moe
from .base import BaseMoeBackend


class FusedMoe(BaseMoeBackend):
    def __init__(self, *args, **kwargs) -> None:
        pass

    def forward(self, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, gating_output: torch.Tensor,
                topk: int, renormalize: bool, activation: str = "silu",
                apply_router_weight_on_input: bool = False) -> torch.Tensor:
        return fused_moe(hidden_states, w1, w2, gating_output, topk, renormalize, activation=activation,
                         apply_router_weight_on_input=apply_router_weight_on_input)
