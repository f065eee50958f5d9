"""MoE backend registry (python/freetoken/moe/__init__.py:16,142-171), reduced to
the hot path: ``fused`` (HBM-resident experts).  The offload slot pool lives in
:mod:`ftmoe.moe.offload_cache`."""
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


def create_moe_backend(backend: str) -> BaseMoeBackend:
    return SUPPORTED_MOE_BACKENDS[backend]()


__all__ = ["BaseMoeBackend", "create_moe_backend", "SUPPORTED_MOE_BACKENDS"]
