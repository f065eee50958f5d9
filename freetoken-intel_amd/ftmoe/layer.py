"""The fused quantized MoE layer (router -> top-k -> grouped w13/act -> w2 ->
deterministic combine, + optional dense shared expert) on gfx950.

:class:`MoeLayer` owns no weights: it references the caller's device banks
(the resident layer, or an :class:`~ftmoe.moe.offload_cache.OffloadMoeCache`
slot pool plus a ``slot_of_expert`` map) and drives ``ftm_moe_forward`` /
``ftm_moe_forward_routed`` on the current HIP stream.

Replaces, for one MoE block:
  * ``_Qwen35MoE.forward`` (python/freetoken/models/qwen3_5_moe/__init__.py:1221-1252)
  * ``_Qwen3MoE.forward`` routing (python/freetoken/models/qwen3_moe/__init__.py:466-541)
  * ``_GptOssMoE.forward`` (python/freetoken/models/gpt_oss/__init__.py:347-365)
  * the per-(token, expert) loop of ``_forward_offload_core``
    (python/freetoken/models/qwen3_5_moe/__init__.py:1706-1737)
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _native as nat
from .banks import Proj

ROUTE_MODES = {
    "softmax_topk": nat.ROUTE_SOFTMAX_TOPK,
    "softmax_topk_lowp": nat.ROUTE_SOFTMAX_TOPK_LOWP,
    "topk_softmax": nat.ROUTE_TOPK_SOFTMAX,
}
ACTIVATIONS = {
    "silu": nat.ACT_SILU,
    "swiglu": nat.ACT_SILU,
    "swish": nat.ACT_SILU,
    "gelu": nat.ACT_GELU,
    "relu": nat.ACT_RELU,
    "swiglu_oai": nat.ACT_SWIGLU_OAI,
}

# One growing workspace per (device, stream): the layer kernels run in stream
# order, so every MoE layer on a stream can share it.  Its control words are
# zero at allocation and every call leaves its counters zero again.
_WS: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, nat.WS_CTRL_BYTES), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


class MoeLayer:
    """Device-resident description of one MoE layer.

    Args:
        w13, w2: routed-expert banks (:class:`~ftmoe.banks.Proj`), ``[S, 2I, H]`` / ``[S, H, I]`` logical.
        num_experts, hidden, inter, topk: E, H, I, k.
        gate_w / gate_b: router weight ``[E, H]`` (bf16) and optional bias ``[E]``.
        shared: optional dict ``{"w13": [2Is, H], "w2": [H, Is], "gate": [1, H]}`` (bf16).
        route_mode: ``"softmax_topk"`` (Qwen3.5, fp32 softmax), ``"softmax_topk_lowp"``
            (softmax in the logits dtype, Qwen3 / ``fused_moe``), ``"topk_softmax"`` (gpt-oss).
        act: ``"silu"`` / ``"gelu"`` / ``"relu"`` / ``"swiglu_oai"``.
        slot_of_expert: optional int32 device tensor ``[E]`` mapping expert -> bank slot.
    """

    def __init__(self, *, w13: Proj, w2: Proj, num_experts: int, hidden: int, inter: int, topk: int,
                 gate_w: Optional[torch.Tensor] = None, gate_b: Optional[torch.Tensor] = None,
                 shared: Optional[dict] = None, route_mode: str = "softmax_topk", renormalize: bool = True,
                 act: str = "silu", swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0,
                 apply_router_weight_on_input: bool = False, slot_of_expert: Optional[torch.Tensor] = None,
                 act_dtype: torch.dtype = torch.bfloat16) -> None:
        if route_mode not in ROUTE_MODES:
            raise ValueError(f"unknown route_mode {route_mode!r}")
        if act not in ACTIVATIONS:
            raise ValueError(f"unsupported MoE activation: {act!r}")
        self.w13, self.w2 = w13, w2
        self.num_experts, self.hidden, self.inter, self.topk = num_experts, hidden, inter, topk
        self.gate_w = gate_w.contiguous() if gate_w is not None else None
        self.gate_b = gate_b.contiguous() if gate_b is not None else None
        self.shared = {k: v.contiguous() for k, v in shared.items()} if shared else None
        self.route_mode, self.renormalize, self.act = route_mode, renormalize, act
        self.swiglu_alpha, self.swiglu_limit = swiglu_alpha, swiglu_limit
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self.slot_of_expert = slot_of_expert
        self.act_dtype = act_dtype
        self.device = w13.device
        for name, t in (("w13", w13.w), ("w2", w2.w), ("gate_w", self.gate_w), ("slot_of_expert", slot_of_expert)):
            nat.require_gpu(t, name)
        self._c: Optional[nat.FtmMoeLayer] = None

    @property
    def shared_inter(self) -> int:
        return int(self.shared["w2"].shape[1]) if self.shared else 0

    def c(self) -> nat.FtmMoeLayer:
        if self._c is None:
            L = nat.FtmMoeLayer()
            L.w13 = self.w13.c()
            L.w2 = self.w2.c()
            L.slot_of_expert = nat.ptr(self.slot_of_expert)
            L.gate_w = nat.ptr(self.gate_w)
            L.gate_b = nat.ptr(self.gate_b)
            if self.shared:
                L.shared_w13 = self.shared["w13"].data_ptr()
                L.shared_w2 = self.shared["w2"].data_ptr()
                L.shared_gate = self.shared["gate"].data_ptr()
            L.num_experts = self.num_experts
            L.hidden = self.hidden
            L.inter = self.inter
            L.topk = self.topk
            L.shared_inter = self.shared_inter
            L.route_mode = ROUTE_MODES[self.route_mode]
            L.renormalize = 1 if self.renormalize else 0
            L.act = ACTIVATIONS[self.act]
            L.swiglu_alpha = float(self.swiglu_alpha)
            L.swiglu_limit = float(self.swiglu_limit)
            L.apply_router_weight_on_input = 1 if self.apply_router_weight_on_input else 0
            L.act_dtype = nat.dtype_code(self.act_dtype)
            self._c = L
        return self._c

    def invalidate(self) -> None:
        """Drop the cached C descriptor (call after swapping bank tensors)."""
        self._c = None

    def workspace_bytes(self, num_tokens: int) -> int:
        return int(nat.lib().ftm_moe_workspace_bytes(ctypes.byref(self.c()), int(num_tokens)))

    def _check_x(self, x: torch.Tensor) -> torch.Tensor:
        nat.require_gpu(x, "hidden_states")
        if x.dim() != 2 or x.shape[1] != self.hidden:
            raise ValueError(f"hidden_states must be [T, {self.hidden}], got {tuple(x.shape)}")
        if x.dtype != self.act_dtype:
            raise TypeError(f"hidden_states dtype {x.dtype} != layer activation dtype {self.act_dtype}")
        return x.contiguous()

    def forward(self, x: torch.Tensor, *, return_routing: bool = False):
        """Whole layer: ``x [T, H] -> out [T, H]`` (routing from ``gate_w``)."""
        x = self._check_x(x)
        T = x.shape[0]
        out = torch.empty_like(x)
        ids = torch.empty((T, self.topk), dtype=torch.int32, device=x.device) if return_routing else None
        w = torch.empty((T, self.topk), dtype=torch.float32, device=x.device) if return_routing else None
        logits = torch.empty((T, self.num_experts), dtype=torch.float32, device=x.device) if return_routing else None
        need = self.workspace_bytes(T)
        ws = workspace(x.device, need)
        rc = nat.lib().ftm_moe_forward(ctypes.byref(self.c()), x.data_ptr(), T, out.data_ptr(), nat.ptr(ids),
                                       nat.ptr(w), nat.ptr(logits), ws.data_ptr(), ws.numel(), nat.stream_of(x))
        nat.check(rc, "ftm_moe_forward")
        if return_routing:
            return out, ids, w, logits
        return out

    def forward_stage(self, x: torch.Tensor, out: torch.Tensor, stage: int,
                      ws: Optional[torch.Tensor] = None) -> None:
        """Launch one stage (``ftmoe._native.STAGE_*``) of :meth:`forward` into ``out``
        (for per-kernel timing; stages 0..4 in order equal one forward).  ``ws``:
        an explicit workspace (uint8, zero-initialised, at least
        :meth:`workspace_bytes`), so several layers' stages can interleave."""
        T = x.shape[0]
        if ws is None:
            ws = workspace(x.device, self.workspace_bytes(T))
        elif ws.numel() < self.workspace_bytes(T):
            raise ValueError("workspace too small")
        rc = nat.lib().ftm_moe_forward_stage(ctypes.byref(self.c()), x.data_ptr(), T, out.data_ptr(), int(stage),
                                             ws.data_ptr(), ws.numel(), nat.stream_of(x))
        nat.check(rc, "ftm_moe_forward_stage")

    def stage_kernel(self, num_tokens: int, stage: int) -> Optional[str]:
        """Base name of the kernel :meth:`forward_stage` launches for ``stage`` at
        ``num_tokens`` tokens (None on the generic path); no device work."""
        name = nat.lib().ftm_moe_stage_kernel(ctypes.byref(self.c()), int(num_tokens), int(stage))
        return name.decode() if name is not None else None

    def forward_routed(self, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor) -> torch.Tensor:
        """Routed experts (+ shared) for caller-supplied routing ``[T, k]``."""
        x = self._check_x(x)
        T = x.shape[0]
        if tuple(topk_ids.shape) != (T, self.topk) or tuple(topk_w.shape) != (T, self.topk):
            raise ValueError(f"routing must be [T, {self.topk}], got {tuple(topk_ids.shape)} / {tuple(topk_w.shape)}")
        nat.require_gpu(topk_ids, "topk_ids")
        nat.require_gpu(topk_w, "topk_w")
        ids = topk_ids.to(torch.int32).contiguous()
        w = topk_w.to(torch.float32).contiguous()
        out = torch.empty_like(x)
        ws = workspace(x.device, self.workspace_bytes(T))
        rc = nat.lib().ftm_moe_forward_routed(ctypes.byref(self.c()), x.data_ptr(), T, ids.data_ptr(), w.data_ptr(),
                                              out.data_ptr(), ws.data_ptr(), ws.numel(), nat.stream_of(x))
        nat.check(rc, "ftm_moe_forward_routed")
        return out

    def route(self, x: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None):
        """Router only: ``(topk_ids int32 [T,k], topk_w f32 [T,k], logits f32 [T,E])``."""
        if logits is not None:
            nat.require_gpu(logits, "gating_output")
            logits = logits.contiguous()
            T = logits.shape[0]
            dev = logits.device
            lin, ldt = logits.data_ptr(), nat.dtype_code(logits.dtype)
            xp = None
        else:
            x = self._check_x(x)
            T, dev, lin, ldt, xp = x.shape[0], x.device, None, 0, x.data_ptr()
        ids = torch.empty((T, self.topk), dtype=torch.int32, device=dev)
        w = torch.empty((T, self.topk), dtype=torch.float32, device=dev)
        lo = torch.empty((T, self.num_experts), dtype=torch.float32, device=dev)
        ws = workspace(dev, self.workspace_bytes(T))
        rc = nat.lib().ftm_route(ctypes.byref(self.c()), xp, T, lin, ldt, lo.data_ptr(), ids.data_ptr(), w.data_ptr(),
                                 ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
        nat.check(rc, "ftm_route")
        return ids, w, lo

    def expert_forward(self, slot: int, x: torch.Tensor) -> torch.Tensor:
        """One expert (bank slot ``slot``) on ``x [M, H]``: down(act(gate(x)) * up(x))."""
        x = self._check_x(x)
        M = x.shape[0]
        out = torch.empty_like(x)
        ws = workspace(x.device, self.workspace_bytes(M))
        rc = nat.lib().ftm_expert_forward(ctypes.byref(self.c()), int(slot), x.data_ptr(), M, out.data_ptr(),
                                          ws.data_ptr(), ws.numel(), nat.stream_of(x))
        nat.check(rc, "ftm_expert_forward")
        return out
