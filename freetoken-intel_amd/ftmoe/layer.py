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
# zero at allocation and every call leaves its counters zero again (the sticky
# error word excepted: check_status reads and clears it).
_WS: dict = {}
# Workspaces a larger call replaced on the same stream.  They stay allocated: a
# HIP graph captured before the growth still holds their addresses.
_WS_RETIRED: dict = {}


def _ws_key(device: torch.device) -> tuple:
    return (device.index, torch.cuda.current_stream(device).cuda_stream)


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """This stream's layer workspace, grown to at least ``nbytes``.  Growing
    allocates, which a HIP graph capture cannot record: size it before the
    capture (run the largest batch once on the capture stream, or call
    :func:`reserve_workspace`)."""
    key = _ws_key(device)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"the MoE layer workspace of this stream would grow to {nbytes} bytes inside a HIP graph capture; "
                "run the largest batch once on the capture stream before capturing, or call "
                "ftmoe.layer.reserve_workspace(device, nbytes)")
        if ws is not None:
            _WS_RETIRED.setdefault(key, []).append(ws)
        ws = torch.zeros(max(nbytes, nat.WS_CTRL_BYTES), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def reserve_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Grow the current stream's workspace to ``nbytes`` now (before a capture)."""
    return workspace(torch.device(device), int(nbytes))


_STATUS_TEXT = {
    nat.WS_ERR_SLOT: "a routed expert had no resident slot: stale slot map (ensure_experts desync); "
                     "its pairs contributed zeros",
    nat.WS_ERR_ID: "an expert id was >= num_experts; its pairs contributed zeros",
    nat.WS_ERR_LIST: "more pairs than tokens were routed to one expert; the extra pairs were dropped",
}


def read_status(device: Optional[torch.device] = None, *, clear: bool = True) -> int:
    """The error bits (``ftmoe._native.WS_ERR_*``) the layer kernels recorded in
    the current stream's workspaces since the last clear (waits for the stream)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    key = _ws_key(device)
    bits = 0
    for ws in [_WS.get(key)] + _WS_RETIRED.get(key, []):
        if ws is None:
            continue
        word = ws[nat.WS_ERROR_OFFSET:nat.WS_ERROR_OFFSET + 4].view(torch.int32)
        bits |= int(word.item())
        if clear:
            word.zero_()
    return bits


def check_status(device: Optional[torch.device] = None, *, layer_id: Optional[int] = None) -> None:
    """Raise for the errors :func:`read_status` reports, and clear them: a
    routed expert without a resident slot raises ``IndexError`` as the
    reference's stale-slot tripwire does
    (python/freetoken/models/qwen3_5_moe/__init__.py:1676-1685); an id >= E
    raises ``ValueError``; a list overflow ``RuntimeError``."""
    bits = read_status(device)
    where = f"layer {layer_id}: " if layer_id is not None else ""
    if bits & nat.WS_ERR_SLOT:
        raise IndexError(where + _STATUS_TEXT[nat.WS_ERR_SLOT])
    if bits & nat.WS_ERR_ID:
        raise ValueError(where + _STATUS_TEXT[nat.WS_ERR_ID])
    if bits & nat.WS_ERR_LIST:
        raise RuntimeError(where + _STATUS_TEXT[nat.WS_ERR_LIST])


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
        act_dtype: dtype of ``x``, ``h`` and the output (bf16 or fp32).
        h_dtype: dtype ``h`` is rounded to before the down projection (None: the
            activation dtype's own); fp16 needs fp32 activations.
    """

    def __init__(self, *, w13: Proj, w2: Proj, num_experts: int, hidden: int, inter: int, topk: int,
                 gate_w: Optional[torch.Tensor] = None, gate_b: Optional[torch.Tensor] = None,
                 shared: Optional[dict] = None, route_mode: str = "softmax_topk", renormalize: bool = True,
                 act: str = "silu", swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0,
                 apply_router_weight_on_input: bool = False, slot_of_expert: Optional[torch.Tensor] = None,
                 act_dtype: torch.dtype = torch.bfloat16, h_dtype: Optional[torch.dtype] = None) -> None:
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
        self.h_dtype = h_dtype
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
            L.h_dtype = nat.dtype_code(self.h_dtype) if self.h_dtype is not None else nat.DT_F32
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

    def forward_routed(self, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, *,
                       check: bool = False) -> torch.Tensor:
        """Routed experts (+ shared) for caller-supplied routing ``[T, k]``.  An id
        < 0 marks a pair without an expert; an expert listed twice for one token
        is applied with the sum of its weights.  ``check``: wait for the call and
        raise (:func:`check_status`) if a routed expert had no resident slot."""
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
        if check:
            check_status(x.device)
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
