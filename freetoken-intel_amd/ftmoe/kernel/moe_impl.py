"""MoE kernel dispatch (python/freetoken/kernel/moe_impl.py:20-46): one entry
point for the ``fused`` backend, served by the gfx950 HIP kernels."""
from __future__ import annotations

import torch

from .fused_moe import fused_moe as _fused_moe_hip


def fused_moe(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, gating: torch.Tensor, topk: int,
              renormalize: bool, activation: str = "silu", apply_router_weight_on_input: bool = False) -> torch.Tensor:
    return _fused_moe_hip(hidden_states, w1, w2, gating, topk, renormalize, activation=activation,
                          apply_router_weight_on_input=apply_router_weight_on_input)
