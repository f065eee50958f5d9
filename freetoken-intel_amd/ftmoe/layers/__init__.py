"""Model-facing layers (python/freetoken/layers/): the MoE layer."""
from .moe import Moe

__all__ = ["Moe"]
