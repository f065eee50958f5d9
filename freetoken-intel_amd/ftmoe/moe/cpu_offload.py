"""Engine-selection hooks of the registry keys ``offload``, ``cpu`` and
``hybrid`` (python/freetoken/moe/__init__.py:149-167, moe/offload.py,
moe/cpu_offload.py).  As in the reference, choosing one tells the engine where
a block's routed experts run; the block does not call the backend's dense
``forward`` but the entry point of that mode:

* ``offload``: :func:`ftmoe.moe.offload_cache.moe_offload_forward` over the
  slot pool (``OffloadMoeCache``);
* ``cpu``: :class:`ftmoe.moe.cpu_executor.CpuMoeExecutor` over the host banks;
* ``hybrid``: :func:`ftmoe.moe.hybrid.moe_hybrid_forward` (CPU || GPU split).

Their ``forward`` raises ``NotImplementedError`` naming that entry point, as
the reference's ``CpuOffloadMoeBackend.forward`` does (cpu_offload.py:31-44).
"""
from __future__ import annotations

from .base import BaseMoeBackend


class _EntryPointHook(BaseMoeBackend):
    entry = ""

    def __init__(self, *args, **kwargs) -> None:
        self.args = args
        self.kwargs = kwargs

    def forward(self, hidden_states, w1, w2, gating_output, topk: int, renormalize: bool, activation: str,
                apply_router_weight_on_input: bool):
        raise NotImplementedError(f"{type(self).__name__}.forward is not this mode's entry point: the block calls "
                                  f"{self.entry} with the router's top_idx/top_w and the layer's banks")


class OffloadMoeBackend(_EntryPointHook):
    entry = "ftmoe.moe.offload_cache.moe_offload_forward"


class CpuOffloadMoeBackend(_EntryPointHook):
    entry = "ftmoe.moe.cpu_executor.CpuMoeExecutor"


class HybridMoeBackend(_EntryPointHook):
    entry = "ftmoe.moe.hybrid.moe_hybrid_forward"


__all__ = ["OffloadMoeBackend", "CpuOffloadMoeBackend", "HybridMoeBackend"]
