"""Engine-side integration: the model's MoE block as one grouped call, and
decode steps captured in HIP graphs.

* :class:`MoeBlock` is the drop-in for the MoE block forwards of the
  reference's Qwen-family models -- ``_Qwen35MoE.forward``
  (python/freetoken/models/qwen3_5_moe/__init__.py:1221-1252) with its
  routed experts in HBM (``_forward_inram``, :1331-1373) or behind the slot
  pool (``_forward_offload`` -> ``_forward_offload_core``, :1375-1391,
  1609-1749), and ``_Qwen3MoE.forward``
  (python/freetoken/models/qwen3_moe/__init__.py:466-541).  The router
  (fp32 or model-dtype softmax, top-k, renorm), the always-on shared expert
  with its sigmoid gate, and every routed (token, expert) pair are the
  layer kernels' launches -- no per-pair Python loop, no ``.item()`` / host
  routing copy on the device-LRU path.
* :class:`MoeGraphRunner` is the analogue of ``XpuGraphRunner``
  (python/freetoken/engine/graph.py:65-124): warm a callable up, capture one
  call of it in a HIP graph, replay it.  Warm-up and capture run on the same
  side stream, because the layer workspace is per stream and must reach its
  size before the capture (a capture cannot allocate it).
"""
from __future__ import annotations

from typing import Callable, Optional

import torch

from .layer import MoeLayer
from .moe.offload_cache import OffloadMoeCache, grouped_layer, moe_offload_forward


class MoeGraphRunner:
    """Capture a sequence of kernel launches once; replay it without the Python
    dispatch that produced them (graph.py:65-124).  ``fn`` must read and write
    only tensors whose addresses stay fixed (static input/output buffers).
    One runner holds one graph.

    Capture a whole decode step (every MoE layer of it) per graph, as the
    reference's runner does: measured on MI355X at C3 T=16, a 48-layer step
    replays at 74.2 us per layer against 75.2 for the same launches eagerly,
    while one graph per layer pays a graph launch on every replay (76.3
    against 73.7)."""

    def __init__(self, warmup_iters: int = 3, device: Optional[torch.device] = None) -> None:
        self.warmup_iters = warmup_iters
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._stream: Optional[torch.cuda.Stream] = None

    @property
    def is_captured(self) -> bool:
        return self._graph is not None

    def capture(self, fn: Callable):
        """Run ``fn`` ``warmup_iters`` times on a side stream, then capture one call
        of it on that stream; returns what the captured call returned (its
        buffers are the ones replays write)."""
        if not torch.cuda.is_available():
            raise RuntimeError("HIP graph capture needs a ROCm GPU; run the step eagerly instead")
        self._stream = torch.cuda.Stream(device=self.device)
        self._stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self._stream):
            for _ in range(self.warmup_iters):
                fn()
        torch.cuda.current_stream(self.device).wait_stream(self._stream)
        torch.cuda.synchronize(self.device)
        self._graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph, stream=self._stream):
            result = fn()
        torch.cuda.synchronize(self.device)
        return result

    def replay(self) -> None:
        if self._graph is None:
            raise RuntimeError("MoeGraphRunner.replay() called before capture()")
        self._graph.replay()


def _t(m):
    """A module's weight, or the tensor itself."""
    return m.weight if hasattr(m, "weight") else m


class MoeBlock:
    """One MoE block of a Qwen-family decoder as grouped HIP calls.

    Args:
        gate: router weight ``[E, H]`` (or an ``nn.Linear``).
        top_k, renormalize: routing (softmax over all experts, top-k, renorm).
        softmax_fp32: ``True`` for Qwen3.5 (``F.softmax(..., dtype=float32)``,
            qwen3_5_moe/__init__.py:1225), ``False`` for Qwen3 / ``fused_moe``
            (softmax in the logits' dtype, qwen3_moe/__init__.py:473-475).
        shared: optional ``(gate_proj [Is, H], up_proj [Is, H], down_proj
            [H, Is], shared_expert_gate [1, H])`` weights or modules
            (qwen3_5_moe/__init__.py:1204-1219,1229,1752-1768).
        w13, w2: in-HBM routed banks (:class:`~ftmoe.banks.Proj`) -- or
        cache, layer_id: a slot pool (:class:`OffloadMoeCache`) holding this
            block's experts as MoE layer ``layer_id``.
        intermediate: the routed experts' intermediate size.
        hybrid_fetch_fraction: slot-pool blocks only -- with ``0 < f < 1`` each
            step splits its routed experts between the host CPU and the GPU
            (:func:`~ftmoe.moe.hybrid.moe_hybrid_forward`, the reference's
            ``hybrid`` backend); ``"auto"`` takes ``f`` from this GPU's
            calibration profile when it recommends ``hybrid`` for the pool's
            format (:mod:`ftmoe.moe.bench_profile`); ``None`` = pure offload.
    """

    def __init__(self, *, gate, top_k: int, intermediate: int, renormalize: bool = True, softmax_fp32: bool = True,
                 shared: Optional[tuple] = None, w13=None, w2=None, cache: Optional[OffloadMoeCache] = None,
                 layer_id: int = 0, act: str = "silu", dtype: torch.dtype = torch.bfloat16,
                 hybrid_fetch_fraction=None) -> None:
        if (cache is None) == (w13 is None or w2 is None):
            raise ValueError("MoeBlock needs either in-HBM banks (w13, w2) or a slot pool (cache)")
        self.gate_w = _t(gate).detach().to(dtype).contiguous()
        self.num_experts, self.hidden = self.gate_w.shape
        self.top_k, self.intermediate, self.dtype = int(top_k), int(intermediate), dtype
        self.cache, self.layer_id, self.act = cache, int(layer_id), act
        self.shared = None
        if shared is not None:
            gp, up, dp, sg = (_t(m).detach().to(dtype) for m in shared)
            self.shared = {"w13": torch.cat([gp, up], dim=0).contiguous(), "w2": dp.contiguous(),
                           "gate": sg.reshape(1, -1).contiguous()}
        if hybrid_fetch_fraction == "auto" and cache is not None:
            from .moe.bench_profile import load_backend_recommendation, load_hybrid_fetch_fraction

            fmt = cache.quant_format
            hybrid_fetch_fraction = (load_hybrid_fetch_fraction(fmt)
                                     if load_backend_recommendation(fmt) == "hybrid" else None)
        elif hybrid_fetch_fraction is not None and cache is None:
            raise ValueError("hybrid_fetch_fraction applies to slot-pool blocks (cache=...) only")
        self.hybrid_fetch_fraction = None if hybrid_fetch_fraction is None else float(hybrid_fetch_fraction)
        mode = "softmax_topk" if softmax_fp32 else "softmax_topk_lowp"
        if cache is None:
            self.layer = MoeLayer(w13=w13, w2=w2, num_experts=self.num_experts, hidden=self.hidden,
                                  inter=self.intermediate, topk=self.top_k, gate_w=self.gate_w, shared=self.shared,
                                  route_mode=mode, renormalize=renormalize, act=act, act_dtype=dtype)
        else:
            # the router alone (ids and weights stay on the GPU), then the pool's grouped layer
            self.router = MoeLayer(w13=_RouterOnly.proj(self.gate_w, self.hidden), w2=_RouterOnly.proj_down(
                self.gate_w, self.hidden), num_experts=self.num_experts, hidden=self.hidden, inter=_RouterOnly.I,
                topk=self.top_k, gate_w=self.gate_w, route_mode=mode, renormalize=renormalize, act_dtype=dtype)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """``routed + sigmoid(x . g_s) * shared(x)`` of ``hidden_states [..., H]``
        (qwen3_5_moe/__init__.py:1221-1252)."""
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        if flat.dtype != self.dtype:
            flat = flat.to(self.dtype)
        if self.cache is None:
            return self.layer.forward(flat).view(shape)
        ids, w, _ = self.router.route(flat)
        f = self.hybrid_fetch_fraction
        if f is not None and 0.0 < f < 1.0:
            from .moe.hybrid import moe_hybrid_forward

            return moe_hybrid_forward(flat, ids, w, self.cache, self.layer_id, intermediate=self.intermediate,
                                      fetch_fraction=f, act=self.act, shared=self.shared).view(shape)
        out = moe_offload_forward(flat, ids, w, self.cache, self.layer_id, intermediate=self.intermediate,
                                  act=self.act, shared=self.shared)
        return out.view(shape)

    __call__ = forward

    def pool_layer(self) -> MoeLayer:
        """The slot pool's grouped layer this block runs (offload blocks only)."""
        if self.cache is None:
            raise RuntimeError("in-HBM block: use .layer")
        return grouped_layer(self.cache, self.layer_id, intermediate=self.intermediate, topk=self.top_k,
                             dtype=self.dtype, act=self.act, shared=self.shared)


class _RouterOnly:
    """Placeholder one-slot bf16 banks for a router-only :class:`MoeLayer`
    (``MoeLayer.route`` never touches them)."""

    I = 8
    _cache: dict = {}

    @classmethod
    def proj(cls, like: torch.Tensor, hidden: int):
        from .banks import Proj

        key = ("w13", like.device, hidden)
        if key not in cls._cache:
            cls._cache[key] = Proj("bf16", torch.zeros(1, 2 * cls.I, hidden, dtype=torch.bfloat16,
                                                       device=like.device), 2 * cls.I, hidden)
        return cls._cache[key]

    @classmethod
    def proj_down(cls, like: torch.Tensor, hidden: int):
        from .banks import Proj

        key = ("w2", like.device, hidden)
        if key not in cls._cache:
            cls._cache[key] = Proj("bf16", torch.zeros(1, hidden, cls.I, dtype=torch.bfloat16, device=like.device),
                                   hidden, cls.I)
        return cls._cache[key]


__all__ = ["MoeBlock", "MoeGraphRunner"]
