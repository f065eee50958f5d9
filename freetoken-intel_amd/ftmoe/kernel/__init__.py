"""Drop-in counterparts of python/freetoken/kernel/triton/* (quantized projections,
dequantizers, fused MoE) backed by the gfx950 HIP library."""
