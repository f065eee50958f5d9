"""Global timestamp-LRU pool of HBM expert slots fed by pinned host banks.

The slot API of python/freetoken/moe/offload_cache.py:218-694
(:class:`OffloadMoeCache`) and its per-slot weight view (:697-1128,
:class:`SlotWeightAccessor`), kept name for name, with the pool on the GPU:

* the LRU bookkeeping (``slot_for_id``, ``id_of_slot``, ``usage``, ``step`` and
  the copy plan ``evict_slots`` / ``src_indices`` / ``num_indices``) lives in
  host memory and is updated by the native ``ftm_lru_ensure`` /
  ``ftm_lru_materialize`` (one C++ pass instead of per-slot ``.item()``
  calls); the policy is the reference's: hits stamp ``usage = step``, the
  misses (ascending expert id) each take the ``argmin (usage, slot)`` victim,
  prefill first takes the lowest free slot;
* the host banks are held in pinned memory and :meth:`copy_missing` enqueues
  the staged rows with ``ftm_copy_slots`` (``hipMemcpyAsync``, contiguous runs
  merged) on a side stream that first waits for the compute stream (a slot
  being overwritten may still be read by earlier work); the compute stream
  then waits on the copy's event, so the next layer forward sees the new
  bytes without a host synchronisation;
* ``slot_of_expert(layer)`` is the device ``int32 [E]`` map the layer kernels
  read (``-1`` = not resident).

A pool on the CPU (``device="cpu"``) keeps the bookkeeping usable for
host-only tests, but :meth:`copy_missing` and every compute path need the GPU.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _native as nat

# Bank names of each format (python/freetoken/moe/offload_cache.py:140-173).
_BANK_SCHEMAS: dict = {
    "bf16": ("gate_up", "down"),
    "gptq_int4": ("qweight_gate_up", "qzeros_gate_up", "scales_gate_up", "qweight_down", "qzeros_down",
                  "scales_down"),
    "fp8_block": ("weight_gate_up", "scale_gate_up", "weight_down", "scale_down"),
    "mxfp4": ("blocks_gate_up", "scales_gate_up", "blocks_down", "scales_down"),
    "int8_channel": ("weight_packed_gate_up", "weight_scale_gate_up", "weight_packed_down", "weight_scale_down"),
    "gguf_kquant": ("raw_gate", "raw_up", "raw_down"),
}

# Banks a format may carry beyond its schema: the per-expert projection biases
# of gpt-oss MXFP4 experts, one row per slot like the weights.  Not in the
# reference, whose pool has no bias component (gpt_oss/__init__.py:46-61).
_OPTIONAL_BANKS: dict = {"mxfp4": ("bias_gate_up", "bias_down")}

# Formats whose expert math the gfx950 kernels implement.
_COMPUTE_FORMATS = ("bf16", "gptq_int4", "fp8_block", "mxfp4", "int8_channel")


def gptq_int4_bytes_per_expert_slot(hidden_size: int, moe_intermediate_size: int, group_size: int, *,
                                    qweight_bytes: int = 4, scale_bytes: int = 2) -> int:
    """Packed bytes of one ``gptq_int4`` expert slot (offload_cache.py:176-215):
    per projection ``[K, N]``: qweight ``K/8 x N`` words, qzeros
    ``ceil(K/g) x N/8`` words, scales ``ceil(K/g) x N``; gate_up has
    ``K = hidden``, ``N = 2 * inter``, down the reverse."""
    if hidden_size <= 0 or moe_intermediate_size <= 0 or group_size <= 0:
        raise ValueError(
            "gptq_int4_bytes_per_expert_slot needs positive hidden_size / "
            "moe_intermediate_size / group_size"
        )

    def proj(k: int, n: int) -> int:
        groups = -(-k // group_size)
        return (k // 8) * n * qweight_bytes + groups * (n // 8) * qweight_bytes + groups * n * scale_bytes

    return proj(hidden_size, 2 * moe_intermediate_size) + proj(moe_intermediate_size, hidden_size)


class OffloadMoeCache:
    """A timestamp-LRU pool of device slots fed by per-layer host expert banks.

    Args:
        num_layers: MoE layers (``L``).
        num_experts: experts per layer (``E``).
        cache_size: device slots (``S >= E``).
        device: the slot pool's device (a ROCm GPU; ``"cpu"`` for bookkeeping only).
        quant_format: bank schema (``_BANK_SCHEMAS`` key).
        prefill_overlap: accepted for signature compatibility.
        decode_only: allow ``cache_size < num_experts`` (a pool that never holds
            a whole layer, e.g. 64 slots for 256 experts); :meth:`materialize_layer`
            then refuses.  Not in the reference, whose pool always fits a layer.
        device_lru: keep the LRU state (``slot_for_id``, ``id_of_slot``,
            ``usage``, ``step``, the plan and the miss counters) in device memory
            and run :meth:`ensure_experts` and :meth:`copy_missing` as GPU kernels
            (``ftm_lru_ensure_dev``, ``ftm_copy_slots_dev``): the routed ids never
            travel to the host, so a decode step is enqueued without a
            synchronisation.  The state after every call equals the host LRU's.
            Out-of-range ids cannot raise at the call; they are ignored and
            recorded for :meth:`check_status`.  Upstream's device-side
            ``lru_ensure`` (offload_cache.py:14-30); the reference port has none.
    """

    def __init__(self, num_layers: int, num_experts: int, cache_size: int, device, quant_format: str = "bf16",
                 prefill_overlap: bool = False, *, decode_only: bool = False, device_lru: bool = False) -> None:
        if quant_format not in _BANK_SCHEMAS:
            raise ValueError(f"unknown quant_format {quant_format!r}")
        self.device_lru = bool(device_lru)
        if self.device_lru and torch.device(device).type != "cuda":
            raise ValueError("device_lru keeps the LRU in GPU memory: the slot pool must live on a GPU")
        if self.device_lru and num_experts > 512:
            raise ValueError(f"device_lru handles at most 512 experts per layer, got {num_experts}")
        self.decode_only = decode_only
        if cache_size < 2 or (cache_size < num_experts and not decode_only):
            raise ValueError(
                f"cache_size {cache_size} must be >= num_experts {num_experts} "
                "(the prefill double buffer borrows the first 2*num_experts slots)"
            )
        self.num_layers = num_layers
        self.num_experts = num_experts
        self.cache_size = cache_size
        self.device = torch.device(device)
        self.quant_format = quant_format
        self.bank_schema = _BANK_SCHEMAS[quant_format]
        self.prefill_overlap = prefill_overlap
        self._alloc_bookkeeping(cache_size)
        self.active_mask = torch.zeros((num_experts,), dtype=torch.int32)
        sdev = self.device if self.device_lru else "cpu"
        self.step = torch.zeros((), dtype=torch.int64, device=sdev)
        self._stats = torch.zeros((2,), dtype=torch.int64, device=sdev)  # misses, calls
        self.stat_missing = self._stats[0]
        self.stat_calls = self._stats[1]
        self._status = torch.zeros((1,), dtype=torch.int32, device=sdev)
        self._max_staged = 0
        self._copy_descs: dict = {}
        self._pool_layers: dict = {}
        self.bank_sources: dict = {}
        self.bank_caches: dict = {}
        self.banks: list = []
        self.extra_metadata: dict = {}
        self._pending_src_layer: Optional[int] = None
        self._pending_whole_layer = False
        self._side_stream = None
        self._copy_done = None
        # device mirror of slot_for_id (host LRU): one buffer for the cache's
        # lifetime, so layer descriptors that hold its address stay valid
        self._slot_dev: Optional[torch.Tensor] = None
        self._slot_dirty = True

    def _alloc_bookkeeping(self, cache_size: int) -> None:
        dev = self.device if self.device_lru else "cpu"
        self.slot_for_id = torch.full((self.num_layers, self.num_experts), -1, dtype=torch.int32, device=dev)
        self.id_of_slot = torch.full((cache_size,), -1, dtype=torch.int32, device=dev)
        self.usage = torch.zeros((cache_size,), dtype=torch.int64, device=dev)
        plan = max(self.num_experts, cache_size)
        self.evict_slots = torch.zeros((plan,), dtype=torch.int32, device=dev)
        self.src_indices = torch.zeros((plan,), dtype=torch.int32, device=dev)
        self.num_indices = torch.zeros((1,), dtype=torch.int64)
        self._staged = torch.zeros((1,), dtype=torch.int32, device=dev)

    # -- bank wiring ---------------------------------------------------------------

    @property
    def is_gpu(self) -> bool:
        return self.device.type == "cuda"

    @property
    def is_xpu(self) -> bool:
        """The reference's accelerator flag (offload_cache.py:691-694): true when
        the pool lives on the accelerator (here a ROCm GPU)."""
        return self.is_gpu

    def set_bank_sources(self, sources: dict) -> None:
        """Attach the host banks (``{bank: [num_layers x [E, ...] host tensor]}``)
        and allocate one ``[cache_size, ...]`` device pool per bank.  Host banks
        are kept in pinned memory (copied there if they are not already)."""
        base, opt = _BANK_SCHEMAS[self.quant_format], _OPTIONAL_BANKS.get(self.quant_format, ())
        extra = set(sources) - set(base)
        if not set(base) <= set(sources) or extra not in (set(), set(opt)):
            raise ValueError(f"banks {sorted(sources)} do not match the {self.quant_format!r} schema {base}"
                             + (f" (optionally with {opt})" if opt else ""))
        self.bank_schema = base + (opt if extra else ())
        self.banks = []
        for bank in self.bank_schema:
            per_layer = sources[bank]
            if len(per_layer) != self.num_layers:
                raise ValueError(f"bank {bank!r} has {len(per_layer)} layers, expected {self.num_layers}")
            hosts = []
            for t in per_layer:
                if t.device.type != "cpu":
                    raise ValueError(f"bank {bank!r}: host sources must live in host memory")
                t = t.contiguous()
                if self.is_gpu and not t.is_pinned():
                    t = t.pin_memory()
                hosts.append(t)
            row_shape = hosts[0].shape[1:]
            cache = torch.zeros((self.cache_size, *row_shape), dtype=hosts[0].dtype, device=self.device)
            self.bank_sources[bank] = hosts
            self.bank_caches[bank] = cache
            self.banks.append((hosts, cache))
        self._copy_descs = {}
        self._pool_layers = {}

    def set_extra_metadata(self, name: str, per_layer: list) -> None:
        if len(per_layer) != self.num_layers:
            raise ValueError(f"extra metadata {name!r} has {len(per_layer)} layers, expected {self.num_layers}")
        self.extra_metadata[name] = list(per_layer)

    def get_extra_metadata(self, name: str, layer_id: int):
        return self.extra_metadata[name][layer_id]

    def rebuild(self, cache_size: int) -> None:
        """Re-allocate the device pool at ``cache_size`` and clear the LRU state
        (offload_cache.py:342-388); the host banks are kept."""
        if cache_size < 2 or (cache_size < self.num_experts and not self.decode_only):
            raise ValueError(f"rebuild cache_size {cache_size} must be >= num_experts {self.num_experts}")
        self.cache_size = cache_size
        self._alloc_bookkeeping(cache_size)
        if self.bank_sources:
            for bank in self.bank_schema:
                hosts = self.bank_sources[bank]
                self.bank_caches[bank] = torch.zeros((cache_size, *hosts[0].shape[1:]), dtype=hosts[0].dtype,
                                                     device=self.device)
            self.banks = [(self.bank_sources[b], self.bank_caches[b]) for b in self.bank_schema]
        self._copy_descs = {}
        self._pool_layers = {}
        self.step.zero_()
        self.active_mask.zero_()
        self._pending_src_layer = None
        self._pending_whole_layer = False
        self._slot_dirty = True

    def bank_views(self, n: Optional[int] = None) -> tuple:
        """Per-bank device pools in schema order: all ``S`` slots, or the first ``n``."""
        if not self.banks:
            raise AssertionError("set_bank_sources must register the banks first")
        if n is None:
            return tuple(cache for _, cache in self.banks)
        return tuple(cache[:n] for _, cache in self.banks)

    # -- reset -------------------------------------------------------------------

    def _resync_slot_for_id(self) -> None:
        """Rebuild ``slot_for_id`` from ``id_of_slot`` (the authoritative map)."""
        E = self.num_experts
        self.slot_for_id.fill_(-1)
        ids = self.id_of_slot.to(torch.int64)
        slots = (ids >= 0).nonzero(as_tuple=True)[0]
        valid = ids[slots]
        self.slot_for_id[valid // E, valid % E] = slots.to(torch.int32)
        self._slot_dirty = True

    def reset(self) -> None:
        self.slot_for_id.fill_(-1)
        self.id_of_slot.fill_(-1)
        self.usage.zero_()
        self.step.zero_()
        self.active_mask.zero_()
        self.num_indices.zero_()
        self._pending_src_layer = None
        self._pending_whole_layer = False
        self._slot_dirty = True
        for cache in self.bank_caches.values():
            cache.zero_()
        self.reset_stats()

    def reset_stats(self) -> None:
        self._stats.zero_()

    def check_status(self) -> None:
        """Raise for the errors recorded on the GPU since the last check (waits
        for the GPU): with ``device_lru``, what the host LRU raises at the call;
        then the layer kernels' error word of the current stream
        (:func:`ftmoe.layer.check_status`: a routed expert without a resident
        slot raises ``IndexError``, the reference's stale-slot tripwire,
        python/freetoken/models/qwen3_5_moe/__init__.py:1676-1685)."""
        if self.device_lru:
            st = int(self._status.item())
            self._status.zero_()
            if st & 1:
                raise ValueError(f"expert ids must lie in [0, {self.num_experts})")
            if st & 2:
                raise RuntimeError("slot_for_id held a slot outside the pool (the expert was reloaded)")
        if self.is_gpu:
            from ..layer import check_status

            check_status(self.device)

    def decode_miss_stats(self) -> dict:
        return {"missing": int(self.stat_missing.item()), "calls": int(self.stat_calls.item())}

    # -- LRU -----------------------------------------------------------------------

    def _lru_args(self):
        # host tensors updated in place by the native LRU
        return (self.slot_for_id.data_ptr(), self.id_of_slot.data_ptr(), self.usage.data_ptr(),
                self.step.data_ptr(), self.evict_slots.data_ptr(), self.src_indices.data_ptr(),
                self._staged.data_ptr())

    def materialize_layer(self, layer_id: int, expert_ids: Optional[torch.Tensor] = None) -> None:
        """Make every expert of ``layer_id`` resident for a prefill forward
        (offload_cache.py:461-556); ``expert_ids`` is accepted and left untouched."""
        if not (0 <= layer_id < self.num_layers):
            raise ValueError(f"Invalid materialize layer id {layer_id}")
        if self.cache_size < self.num_experts:
            raise ValueError(f"cache_size {self.cache_size} < num_experts {self.num_experts}: "
                             "cannot materialize a whole layer")
        self.active_mask.fill_(1)
        if self.device_lru:  # prefill is rare: plan on the host copies, then put the state back
            host = [t.cpu() for t in (self.slot_for_id, self.id_of_slot, self.usage, self.step, self.evict_slots,
                                      self.src_indices, self._staged)]
            rc = nat.lib().ftm_lru_materialize(layer_id, self.num_layers, self.num_experts, self.cache_size,
                                               *(t.data_ptr() for t in host))
            nat.check(rc, "ftm_lru_materialize")
            for dst, src in zip((self.slot_for_id, self.id_of_slot, self.usage, self.step, self.evict_slots,
                                 self.src_indices, self._staged), host):
                dst.copy_(src)
            staged = int(host[-1][0])
            self._stats += torch.tensor([staged, 1], dtype=torch.int64, device=self.device)
            self._max_staged = staged
            self.num_indices.fill_(staged)
            self._pending_src_layer = layer_id
            self._pending_whole_layer = True
            return
        rc = nat.lib().ftm_lru_materialize(layer_id, self.num_layers, self.num_experts, self.cache_size,
                                           *self._lru_args())
        nat.check(rc, "ftm_lru_materialize")
        self._after_plan(layer_id, int(self._staged[0]), whole=True)

    def ensure_experts(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        """Make this layer's routed experts resident (offload_cache.py:560-647):
        hits keep their slots, each miss evicts the global LRU slot and is
        staged for :meth:`copy_missing`.  ``expert_ids`` is read (a device
        tensor is copied to the host) and never rewritten."""
        if not (0 <= layer_id < self.num_layers):
            raise ValueError(f"Invalid layer id {layer_id}")
        if self.banks and self.cache_size < 2:
            raise RuntimeError(
                f"cache_size {self.cache_size} < 2: the pool cannot hold a routed expert plus "
                "a victim to evict; raise moe_cache_size"
            )
        if self.device_lru:
            self.ensure_experts_chunk(layer_id, expert_ids, 0, self.num_experts)
            return
        ids = expert_ids.reshape(-1).to("cpu", torch.int64).contiguous()
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.num_experts):
            raise ValueError(f"expert ids must lie in [0, {self.num_experts})")
        self.active_mask.zero_()
        if ids.numel():
            self.active_mask[ids] = 1
        rc = nat.lib().ftm_lru_ensure(layer_id, self.num_layers, self.num_experts, self.cache_size,
                                      ids.data_ptr() if ids.numel() else None, int(ids.numel()),
                                      *self._lru_args())
        nat.check(rc, "ftm_lru_ensure")
        self._after_plan(layer_id, int(self._staged[0]), whole=False)

    def ensure_experts_chunk(self, layer_id: int, expert_ids: torch.Tensor, chunk: int, chunk_cap: int,
                             want_ids: bool = False) -> Optional[torch.Tensor]:
        """``device_lru``: :meth:`ensure_experts` for the routed experts of ranks
        ``[chunk * chunk_cap, (chunk + 1) * chunk_cap)`` in ascending id (chunk 0
        is always an LRU step; a later chunk past the last routed expert changes
        nothing), on the current stream.  ``want_ids``: also return
        ``expert_ids`` with every pair outside the chunk set to -1 (int32, same
        shape).  Ids < 0 are pairs without an expert."""
        if not self.device_lru:
            raise RuntimeError("ensure_experts_chunk runs the device LRU (device_lru=True)")
        if not (0 <= layer_id < self.num_layers):
            raise ValueError(f"Invalid layer id {layer_id}")
        if self.banks and self.cache_size < 2:
            raise RuntimeError(
                f"cache_size {self.cache_size} < 2: the pool cannot hold a routed expert plus "
                "a victim to evict; raise moe_cache_size"
            )
        ids = expert_ids.to(self.device, torch.int32).contiguous()
        n = ids.numel()
        ids_c = torch.empty_like(ids) if want_ids else None
        rc = nat.lib().ftm_lru_ensure_dev(
            layer_id, self.num_layers, self.num_experts, self.cache_size, ids.data_ptr() if n else None, n,
            int(chunk), int(chunk_cap), self.slot_for_id.data_ptr(), self.id_of_slot.data_ptr(),
            self.usage.data_ptr(), self.step.data_ptr(), self.evict_slots.data_ptr(), self.src_indices.data_ptr(),
            self._staged.data_ptr(), ids_c.data_ptr() if ids_c is not None else None, self._stats.data_ptr(),
            self._status.data_ptr(), torch.cuda.current_stream(self.device).cuda_stream)
        nat.check(rc, "ftm_lru_ensure_dev")
        self._max_staged = min(self.num_experts, int(chunk_cap), n)
        self._pending_src_layer = layer_id
        self._pending_whole_layer = False
        return ids_c

    def _after_plan(self, layer_id: int, staged: int, whole: bool) -> None:
        self.num_indices.fill_(staged)
        self.stat_missing += staged
        self.stat_calls += 1
        self._pending_src_layer = layer_id
        self._pending_whole_layer = whole
        self._slot_dirty = True

    # -- copy engine -----------------------------------------------------------------

    def copy_missing(self) -> None:
        """Stream the staged (slot, host row) pairs of every bank into the device
        pools on a side stream (pinned host -> HBM), ordered after the work
        already queued on the current stream, and make the current stream wait
        for the copies."""
        if not self.banks:
            raise AssertionError("set_bank_sources must register the banks first")
        layer_id = self._pending_src_layer
        if layer_id is None:
            return
        if not self.is_gpu:
            raise RuntimeError("copy_missing streams into a GPU slot pool; this cache lives on the CPU")
        if self.device_lru:
            # the plan stays in device memory: one kernel reads it and pulls the rows of every bank
            descs = self._copy_descs.get(layer_id)
            if descs is None:
                descs = (nat.FtmBankCopy * len(self.banks))()
                for j, (hosts, cache) in enumerate(self.banks):
                    host = hosts[layer_id]
                    descs[j] = nat.FtmBankCopy(host.data_ptr(), cache.data_ptr(), host[0].numel() * host.element_size())
                self._copy_descs[layer_id] = descs
            if self._max_staged:
                rc = nat.lib().ftm_copy_slots_dev(descs, len(self.banks), self.num_experts, self.cache_size,
                                                  self.evict_slots.data_ptr(), self.src_indices.data_ptr(),
                                                  self._staged.data_ptr(), self._max_staged,
                                                  torch.cuda.current_stream(self.device).cuda_stream)
                nat.check(rc, "ftm_copy_slots_dev")
            self._pending_src_layer = None
            self._pending_whole_layer = False
            return
        n = int(self.num_indices.item())
        if n:
            cur = torch.cuda.current_stream(self.device)
            if self._side_stream is None:
                self._side_stream = torch.cuda.Stream(device=self.device)
                self._copy_done = torch.cuda.Event()
            side = self._side_stream
            side.wait_stream(cur)
            for hosts, cache in self.banks:
                host = hosts[layer_id]
                row_bytes = host[0].numel() * host.element_size()
                rc = nat.lib().ftm_copy_slots(cache.data_ptr(), host.data_ptr(), row_bytes,
                                              self.evict_slots.data_ptr(), self.src_indices.data_ptr(), n,
                                              side.cuda_stream, None)
                nat.check(rc, "ftm_copy_slots")
            self._copy_done.record(side)
            cur.wait_event(self._copy_done)
        self._pending_src_layer = None
        self._pending_whole_layer = False

    # -- device helpers ----------------------------------------------------------------

    def slot_of_expert(self, layer_id: int) -> torch.Tensor:
        """Device ``int32 [E]``: the slot holding each expert of ``layer_id``, -1 if
        not resident (what the layer kernels read)."""
        if self.device_lru:
            return self.slot_for_id[layer_id]
        if self._slot_dev is None:
            self._slot_dev = torch.full_like(self.slot_for_id, -1, device=self.device)
            self._slot_dirty = True
        if self._slot_dirty:
            # a pinned snapshot: the host map changes again before the copy runs
            src = self.slot_for_id.pin_memory() if self.is_gpu else self.slot_for_id
            self._slot_dev.copy_(src, non_blocking=True)
            self._slot_dirty = False
        return self._slot_dev[layer_id]

    def require_resident(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        """Host LRU: raise ``IndexError`` when a routed expert of ``layer_id`` has
        no slot in ``[0, cache_size)`` -- the reference's loud stale-slot guard
        (python/freetoken/models/qwen3_5_moe/__init__.py:1676-1685), here also
        for a slot of -1 (the reference would skip such a pair silently)."""
        if self.device_lru:
            raise RuntimeError("require_resident reads the host LRU; with device_lru use check_status()")
        ids = expert_ids.reshape(-1).to("cpu", torch.int64)
        ids = ids[ids >= 0]
        if ids.numel() == 0:
            return
        slots = self.slot_for_id[layer_id].to(torch.int64)[ids]
        bad = (slots < 0) | (slots >= self.cache_size)
        if bool(bad.any()):
            stale = int(slots[bad][0])
            raise IndexError(f"layer {layer_id}: offload routed slot id {stale} outside cache_size "
                             f"{self.cache_size}: stale slot map (ensure_experts desync)")

    def resident_slots(self, layer_id: int) -> list:
        E = self.num_experts
        base = layer_id * E
        ids = self.id_of_slot.cpu()
        return [s for s in range(self.cache_size) if base <= int(ids[s]) < base + E]


class SlotWeightAccessor:
    """Per-slot expert weights of one MoE layer over an :class:`OffloadMoeCache`
    pool (offload_cache.py:697-1128): packed views (``get_*_packed``), dense
    dequantized ``(gate [I, H], up [I, H], down [H, I])`` (:meth:`get`, the GPU
    dequant kernel, cached per instance) and :meth:`expert_forward` (the fused
    gfx950 expert kernel up to the format's crossover, dequant + matmul above).

    Args:
        cache: the slot pool (its banks must be registered).
        intermediate: ``I`` (moe_intermediate_size).
        dtype: the activation dtype (the dequant output dtype).
        layer_id: accepted for signature compatibility (``gguf_kquant`` only).
    """

    def __init__(self, cache: OffloadMoeCache, intermediate: int, dtype: torch.dtype, *,
                 layer_id: Optional[int] = None) -> None:
        self.quant_format = getattr(cache, "quant_format", "bf16")
        self._intermediate = int(intermediate)
        self._dtype = dtype
        self._cache_obj = cache
        self._cache: dict = {}
        self._layer = None
        fmt = self.quant_format
        if fmt not in _COMPUTE_FORMATS:
            raise ValueError(f"SlotWeightAccessor: quant_format {fmt!r} has no gfx950 kernel in this build")
        self._banks = dict(zip(cache.bank_schema, cache.bank_views()))
        if fmt == "gptq_int4":
            group_size = getattr(cache, "gptq_group_size", None)
            if group_size is None:
                raise ValueError(
                    "OffloadMoeCache.gptq_group_size is not set -- the loader must set it "
                    "from the checkpoint's quantization_config.group_size before any "
                    "gptq_int4 forward pass runs (SlotWeightAccessor refuses to guess)"
                )
            self._group_size = int(group_size)
        elif fmt == "fp8_block":
            self._fp8_block = int(getattr(cache, "fp8_block_size", None) or 128)
        elif fmt == "int8_channel":
            k_gate_up = getattr(cache, "int8_k_gate_up", None)
            k_down = getattr(cache, "int8_k_down", None)
            if k_gate_up is None or k_down is None:
                raise ValueError(
                    "OffloadMoeCache.int8_k_gate_up / int8_k_down are not set -- the loader "
                    "must set them from the checkpoint's real weight_shape before any "
                    "int8_channel forward pass runs (SlotWeightAccessor refuses to guess)"
                )
            self._int8_k_gate_up = int(k_gate_up)
            self._int8_k_down = int(k_down)
        if fmt == "bf16":
            self._gu, self._dn = cache.bank_views()

    # -- packed views ----------------------------------------------------------------

    def _require(self, fmt: str, what: str) -> None:
        if self.quant_format != fmt:
            raise ValueError(f"{what} is {fmt}-only, got quant_format={self.quant_format!r}")

    def get_gptq_packed(self, s_i: int):
        self._require("gptq_int4", "get_gptq_packed")
        b = self._banks
        return (b["qweight_gate_up"][s_i], b["qzeros_gate_up"][s_i], b["scales_gate_up"][s_i],
                b["qweight_down"][s_i], b["qzeros_down"][s_i], b["scales_down"][s_i], self._group_size)

    def get_fp8_packed(self, s_i: int):
        self._require("fp8_block", "get_fp8_packed")
        b = self._banks
        return (b["weight_gate_up"][s_i], b["scale_gate_up"][s_i], b["weight_down"][s_i], b["scale_down"][s_i],
                self._fp8_block)

    def get_mxfp4_packed(self, s_i: int):
        self._require("mxfp4", "get_mxfp4_packed")
        b = self._banks
        return (b["blocks_gate_up"][s_i], b["scales_gate_up"][s_i], b["blocks_down"][s_i], b["scales_down"][s_i])

    def get_int8_packed(self, s_i: int):
        self._require("int8_channel", "get_int8_packed")
        b = self._banks
        return (b["weight_packed_gate_up"][s_i], b["weight_scale_gate_up"][s_i], b["weight_packed_down"][s_i],
                b["weight_scale_down"][s_i], self._int8_k_gate_up, self._int8_k_down)

    # -- the pool as one MoE layer (expert = slot) -----------------------------------

    def _hidden(self) -> int:
        b, fmt = self._banks, self.quant_format
        if fmt == "bf16":
            return int(self._gu.shape[-1])
        if fmt == "fp8_block":
            return int(b["weight_gate_up"].shape[-1])
        if fmt == "gptq_int4":
            return int(b["qweight_gate_up"].shape[1]) * 8
        if fmt == "int8_channel":
            return self._int8_k_gate_up
        return int(b["blocks_gate_up"].shape[2]) * 32  # mxfp4

    def pool_layer(self):
        """The slot pool as a :class:`~ftmoe.layer.MoeLayer` whose expert ``s`` is
        slot ``s`` (no router): what :meth:`expert_forward` runs on."""
        if self._layer is None:
            from ..banks import proj_from_bank
            from ..layer import MoeLayer

            I, H, fmt = self._intermediate, self._hidden(), self.quant_format
            group = {"gptq_int4": getattr(self, "_group_size", None), "fp8_block": getattr(self, "_fp8_block", None),
                     "mxfp4": 32}.get(fmt)
            kd = self._int8_k_down if fmt == "int8_channel" else I
            b13, b2 = self._banks.get("bias_gate_up"), self._banks.get("bias_down")  # per slot, MXFP4 only
            w13 = proj_from_bank(fmt, self._banks, which="gate_up", N=2 * I, K=H, group=group, bias=b13)
            w2 = proj_from_bank(fmt, self._banks, which="down", N=H, K=kd, group=group, bias=b2)
            self._layer = MoeLayer(w13=w13, w2=w2, num_experts=w13.num_slots, hidden=H, inter=I, topk=1,
                                   act_dtype=self._dtype)
        return self._layer

    def expert_forward(self, s_i: int, x: torch.Tensor) -> torch.Tensor:
        """``down(silu(gate(x)) * up(x))`` for slot ``s_i`` (offload_cache.py:926-996)
        on the gfx950 expert kernels for every row count: up to the format's
        ``prefer_fused_over_dequant`` crossover the decode stages, above it the
        MFMA-tiled stages the layer switches to (weights decoded exactly in
        registers), where the reference dequantizes the slot with :meth:`get`
        and runs dense matmuls.  fp32 accumulation, ``h`` rounded to the
        accessor's dtype."""
        nat.require_gpu(x, "x")
        return self.pool_layer().expert_forward(int(s_i), x.to(self._dtype))

    def get(self, s_i: int):
        """``(gate_w [I, H], up_w [I, H], down_w [H, I])`` of slot ``s_i`` in the
        accessor's dtype, dequantized once per instance by the GPU kernel."""
        I = self._intermediate
        if self.quant_format == "bf16":
            return self._gu[s_i, 0:I], self._gu[s_i, I:2 * I], self._dn[s_i]
        cached = self._cache.get(s_i)
        if cached is not None:
            return cached
        from ..kernel._dequant import dequant

        layer = self.pool_layer()
        gu = dequant(layer.w13, out_dtype=self._dtype, slot=int(s_i))
        dn = dequant(layer.w2, out_dtype=self._dtype, slot=int(s_i))
        result = (gu[0:I], gu[I:2 * I], dn)
        self._cache[s_i] = result
        return result


def grouped_layer(cache: OffloadMoeCache, layer_id: int, *, intermediate: int, topk: int, dtype: torch.dtype,
                  act: str = "silu", shared: Optional[dict] = None, swiglu_alpha: float = 1.702,
                  swiglu_limit: float = 7.0):
    """The :class:`~ftmoe.layer.MoeLayer` over the slot pool for ``layer_id``
    (expert ``e`` read from slot ``slot_of_expert(layer_id)[e]``), built once per
    (layer, shape, activation, shared expert) and bank registration, so a
    decode step pays no descriptor construction."""
    skey = None if not shared else tuple(sorted((k, v.data_ptr(), tuple(v.shape)) for k, v in shared.items()))
    key = ("grouped", int(layer_id), int(intermediate), dtype, int(topk), act, skey, float(swiglu_alpha),
           float(swiglu_limit))
    layer = cache._pool_layers.get(key)
    if layer is None:
        pkey = (int(intermediate), dtype)
        pool = cache._pool_layers.get(pkey)
        if pool is None:  # the pool's projections, built once per bank registration
            pool = SlotWeightAccessor(cache, intermediate, dtype).pool_layer()
            cache._pool_layers[pkey] = pool
        from ..layer import MoeLayer

        layer = MoeLayer(w13=pool.w13, w2=pool.w2, num_experts=cache.num_experts, hidden=pool.hidden,
                         inter=intermediate, topk=int(topk), shared=shared, act=act, swiglu_alpha=swiglu_alpha,
                         swiglu_limit=swiglu_limit, slot_of_expert=cache.slot_of_expert(layer_id), act_dtype=dtype)
        cache._pool_layers[key] = layer
    else:
        cache.slot_of_expert(layer_id)  # refresh the device map if the host LRU moved
    return layer


def moe_grouped_forward(flat: torch.Tensor, top_idx: torch.Tensor, top_w: torch.Tensor, cache: OffloadMoeCache,
                        layer_id: int, *, intermediate: int, act: str = "silu", shared: Optional[dict] = None,
                        swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0, check: bool = False) -> torch.Tensor:
    """One grouped call for a layer whose experts sit in the slot pool: replaces
    the per-(token, expert) loop of ``_forward_offload_core``
    (python/freetoken/models/qwen3_5_moe/__init__.py:1706-1737).  ``top_idx`` /
    ``top_w`` ``[T, k]`` are expert ids and router weights; the layer must have
    been made resident with :meth:`OffloadMoeCache.ensure_experts` and
    :meth:`~OffloadMoeCache.copy_missing`.  A routed expert that is not
    resident contributes zeros and sets the workspace error bit, which
    ``check=True`` (a synchronisation) or a later :meth:`OffloadMoeCache.check_status`
    turns into ``IndexError``."""
    layer = grouped_layer(cache, layer_id, intermediate=intermediate, topk=int(top_idx.shape[1]), dtype=flat.dtype,
                          act=act, shared=shared, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)
    return layer.forward_routed(flat, top_idx, top_w, check=check)


def moe_offload_forward(flat: torch.Tensor, top_idx: torch.Tensor, top_w: torch.Tensor, cache: OffloadMoeCache,
                        layer_id: int, *, intermediate: int, act: str = "silu", shared: Optional[dict] = None,
                        swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0,
                        ids_host: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The offload decode step of ``_forward_offload_core``
    (python/freetoken/models/qwen3_5_moe/__init__.py:1609-1749) as grouped calls:
    make the routed experts resident (:meth:`OffloadMoeCache.ensure_experts`,
    :meth:`~OffloadMoeCache.copy_missing` on the side stream) and run
    :func:`moe_grouped_forward` over them.

    A step that routes to more experts than the pool holds (a ``decode_only``
    pool) runs in chunks of at most ``cache_size`` experts, in ascending expert
    id: each chunk's pairs keep their ids, the others are passed as -1 (no
    expert), the shared expert rides with the first chunk, and the chunk
    outputs are summed in fp32 and rounded once.  Every routed pair is
    computed; against a single call the chunked sum differs only by the
    rounding of each chunk's output to the activation dtype.  ``ids_host``: a
    host copy of ``top_idx`` when the caller has one (saves the device read
    the LRU planning needs).

    With ``cache.device_lru`` the planning runs on the GPU and nothing is read
    back: the number of distinct experts is not known on the host, so the step
    runs ``ceil(min(T*k, E) / cache_size)`` chunk calls (ranks ``[c * S,
    (c + 1) * S)``; a chunk past the last distinct expert changes nothing and
    adds zeros).  The result and the LRU state equal the host path's."""
    if cache.device_lru:
        cap = cache.cache_size
        ids32 = top_idx.to(torch.int32)
        nchunks = max(1, -(-min(ids32.numel(), cache.num_experts) // cap))
        if nchunks == 1:
            cache.ensure_experts_chunk(layer_id, ids32, 0, cap)
            cache.copy_missing()
            return moe_grouped_forward(flat, top_idx, top_w, cache, layer_id, intermediate=intermediate, act=act,
                                       shared=shared, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)
        acc = None
        for c in range(nchunks):
            ids_c = cache.ensure_experts_chunk(layer_id, ids32, c, cap, want_ids=True)
            cache.copy_missing()
            out_c = moe_grouped_forward(flat, ids_c, top_w, cache, layer_id, intermediate=intermediate, act=act,
                                        shared=shared if c == 0 else None, swiglu_alpha=swiglu_alpha,
                                        swiglu_limit=swiglu_limit)
            acc = out_c.float() if acc is None else acc + out_c.float()
        return acc.to(flat.dtype)
    ids_host = (top_idx if ids_host is None else ids_host).reshape(-1).to("cpu", torch.int64)
    uniq = torch.unique(ids_host)
    uniq = uniq[uniq >= 0]  # ids < 0: pairs without an expert
    cap = cache.cache_size
    if uniq.numel() <= cap:
        cache.ensure_experts(layer_id, uniq)
        cache.require_resident(layer_id, uniq)
        cache.copy_missing()
        return moe_grouped_forward(flat, top_idx, top_w, cache, layer_id, intermediate=intermediate, act=act,
                                   shared=shared, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)
    ids_dev = top_idx.to(torch.int32)
    acc = None
    for c0 in range(0, uniq.numel(), cap):
        chunk = uniq[c0:c0 + cap]
        cache.ensure_experts(layer_id, chunk)
        cache.require_resident(layer_id, chunk)
        cache.copy_missing()
        member = torch.isin(ids_dev, chunk.to(ids_dev.device, torch.int32))
        ids_c = torch.where(member, ids_dev, torch.full_like(ids_dev, -1))
        out_c = moe_grouped_forward(flat, ids_c, top_w, cache, layer_id, intermediate=intermediate, act=act,
                                    shared=shared if c0 == 0 else None, swiglu_alpha=swiglu_alpha,
                                    swiglu_limit=swiglu_limit)
        acc = out_c.float() if acc is None else acc + out_c.float()
    return acc.to(flat.dtype)


__all__ = ["OffloadMoeCache", "SlotWeightAccessor", "_BANK_SCHEMAS", "gptq_int4_bytes_per_expert_slot",
           "grouped_layer", "moe_grouped_forward", "moe_offload_forward"]
