"""MoE backend registry (python/freetoken/moe/__init__.py:16,142-171): ``fused``
(HBM-resident experts, the dense plugin contract) and the engine-selection
hooks ``offload``, ``cpu`` and ``hybrid`` (:mod:`ftmoe.moe.cpu_offload`), whose
entry points are the slot pool's :func:`~ftmoe.moe.offload_cache.moe_offload_forward`,
:class:`~ftmoe.moe.cpu_executor.CpuMoeExecutor` and
:func:`~ftmoe.moe.hybrid.moe_hybrid_forward`."""
from __future__ import annotations

from typing import Callable, Dict

from .base import BaseMoeBackend


class Registry(dict):
    def __init__(self, name: str):
        super().__init__()
        self.name = name

    def register(self, key: str) -> Callable:
        def deco(fn):
            self[key] = fn
            return fn
        return deco

    def __getitem__(self, key):
        if key not in self:
            raise KeyError(f"{self.name} {key!r} is not registered (have {sorted(self.keys())})")
        return super().__getitem__(key)


SUPPORTED_MOE_BACKENDS: Dict[str, Callable[[], BaseMoeBackend]] = Registry("MoE Backend")


@SUPPORTED_MOE_BACKENDS.register("fused")
def create_fused_moe_backend():
    from .fused import FusedMoe

    return FusedMoe()


@SUPPORTED_MOE_BACKENDS.register("offload")
def create_offload_moe_backend():
    from .cpu_offload import OffloadMoeBackend

    return OffloadMoeBackend()


@SUPPORTED_MOE_BACKENDS.register("cpu")
def create_cpu_moe_backend():
    from .cpu_offload import CpuOffloadMoeBackend

    return CpuOffloadMoeBackend()


@SUPPORTED_MOE_BACKENDS.register("hybrid")
def create_hybrid_moe_backend():
    from .cpu_offload import HybridMoeBackend

    return HybridMoeBackend()


def create_moe_backend(backend: str) -> BaseMoeBackend:
    return SUPPORTED_MOE_BACKENDS[backend]()


__all__ = ["BaseMoeBackend", "create_moe_backend", "SUPPORTED_MOE_BACKENDS"]
