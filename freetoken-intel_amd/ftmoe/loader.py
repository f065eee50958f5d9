"""Checkpoint -> packed per-layer expert banks in the layouts the gfx950 kernels read.

The loader side of the reference's offload path
(python/freetoken/models/weight.py:179-269, 745-1600 and
python/freetoken/models/loader.py:693-925), restated for this build:

* format detection from the checkpoint's own ``config.json``
  (``quantization_config.quant_method``; compressed-tensors ``pack-quantized``
  8-bit int for INT8) -- :func:`checkpoint_quant_method` and friends;
* one streaming pass over the safetensors shards that keeps every tensor in
  its packed form and finalizes each ``(layer, gate_up | down)`` bank the
  moment its last component arrives, so no more than one layer's raw
  per-expert tensors are ever buffered -- :func:`stream_moe_expert_sources_gptq`
  / ``_fp8`` / ``_int8`` / ``_mxfp4`` with the reference's bank types
  (:class:`GptqExpertBank`, :class:`Fp8BlockExpertBank`,
  :class:`Int8ExpertBank`, :class:`MxfpExpertBank`) and its errors
  (``ValueError`` for an unknown key, a duplicate or late component, a
  missing expert, misaligned FP8 blocks, inconsistent INT8 ``K``);
* gate and up fused into one ``[2I, ...]`` bank, gate rows first (the
  kernels' ``w13`` convention): GPTQ along its N axis (dim 1 of ``[K/8, N]``),
  FP8 and INT8 along dim 0;
* gpt-oss MXFP4 checkpoints store ``gate_up_proj`` already fused but with
  gate and up rows interleaved (row ``2i`` = gate channel ``i``, row ``2i+1``
  = up channel ``i``) and carry ``gate_up_proj_bias`` / ``down_proj_bias``;
  the reference loader ignores both (a documented scope cut,
  python/freetoken/models/gpt_oss/__init__.py:46-58).  Here the interleaved
  rows (blocks, scales, bias) are split into gate-then-up order and the biases
  ride with the banks;
* :func:`attach_offload_cache` wires the banks into an
  :class:`~ftmoe.moe.offload_cache.OffloadMoeCache` with the attributes the
  slot API reads (``gptq_group_size``, ``int8_k_gate_up`` / ``int8_k_down``,
  ``fp8_block_size``; MXFP4 biases as two more per-slot banks), and
  :func:`moe_layer_from_banks` builds the in-HBM :class:`~ftmoe.layer.MoeLayer`
  of one layer from them.
"""
from __future__ import annotations

import glob
import json
import os
from dataclasses import dataclass
from typing import Callable, Dict, Iterator, Optional, Tuple

import torch

# --------------------------------------------------------------------------- bank types


@dataclass(frozen=True)
class GptqExpertBank:
    """One layer's packed GPTQ bank for one projection (weight.py:745-772).
    ``g_idx`` is shared by every expert of the projection (``k // group_size``)."""

    qweight: torch.Tensor  # [E, K // 8, N] int32
    qzeros: torch.Tensor   # [E, ceil(K / g), N // 8] int32
    scales: torch.Tensor   # [E, ceil(K / g), N]
    g_idx: torch.Tensor    # [K] int32


@dataclass(frozen=True)
class Fp8BlockExpertBank:
    """One layer's block-FP8 bank for one projection (weight.py:981-1007)."""

    weight: torch.Tensor            # [E, N, K] float8_e4m3fn
    weight_scale_inv: torch.Tensor  # [E, ceil(N / B), ceil(K / B)]


@dataclass(frozen=True)
class MxfpExpertBank:
    """One layer's MXFP4 bank for one projection (weight.py:1202-1228), plus the
    per-expert bias gpt-oss checkpoints carry (``None`` when absent)."""

    blocks: torch.Tensor  # [E, N, K // 32, 16] uint8
    scales: torch.Tensor  # [E, N, K // 32] uint8 (e8m0)
    bias: Optional[torch.Tensor] = None  # [E, N] (bf16 in gpt-oss)


@dataclass(frozen=True)
class Int8ExpertBank:
    """One layer's compressed-tensors pack-quantized INT8 bank for one
    projection (weight.py:1352-1394); ``k`` = the logical in-features."""

    weight_packed: torch.Tensor  # [E, N, ceil(K / 4)] int32
    weight_scale: torch.Tensor   # [E, N, num_groups]
    k: int


# --------------------------------------------------------------------------- checkpoint config


def _raw_config(model_path: str) -> dict:
    with open(os.path.join(model_path, "config.json")) as f:
        return json.load(f)


def _quant_config(model_path: str) -> Optional[dict]:
    raw = _raw_config(model_path)
    qc = raw.get("quantization_config")
    if not isinstance(qc, dict):
        text = raw.get("text_config")
        qc = text.get("quantization_config") if isinstance(text, dict) else None
    return qc if isinstance(qc, dict) else None


def checkpoint_quant_method(model_path: str) -> Optional[str]:
    """``quantization_config.quant_method`` of the checkpoint's ``config.json``
    (top level or under ``text_config``), ``None`` when unquantized
    (weight.py:272-296)."""
    qc = _quant_config(model_path)
    return qc.get("quant_method") if qc else None


def _compressed_tensors_weights(model_path: str) -> Optional[dict]:
    qc = _quant_config(model_path)
    groups = qc.get("config_groups") if qc else None
    if not isinstance(groups, dict) or not groups:
        return None
    group = next(iter(groups.values()))
    if not isinstance(group, dict) or group.get("format") != "pack-quantized":
        return None
    w = group.get("weights")
    return w if isinstance(w, dict) else None


def checkpoint_is_int8_pack_quantized(model_path: str) -> bool:
    """compressed-tensors ``pack-quantized`` with 8-bit int weights (weight.py:322-340)."""
    w = _compressed_tensors_weights(model_path)
    return w is not None and w.get("num_bits") == 8 and w.get("type") == "int"


def checkpoint_int8_pack_quantized_group_size(model_path: str) -> Optional[int]:
    """Its ``group_size``; ``None`` = per-channel (weight.py:343-353)."""
    w = _compressed_tensors_weights(model_path)
    return w.get("group_size") if w is not None else None


def checkpoint_gptq_group_size(model_path: str) -> int:
    """``quantization_config.group_size`` of a GPTQ checkpoint (weight.py:356-369)."""
    qc = _quant_config(model_path)
    if not qc or "group_size" not in qc:
        raise ValueError(f"{model_path!r} has no quantization_config.group_size (not a GPTQ checkpoint?)")
    return int(qc["group_size"])


def checkpoint_fp8_block(model_path: str) -> int:
    """Block edge of a block-FP8 checkpoint (``weight_block_size``, square); 128 by default."""
    qc = _quant_config(model_path) or {}
    wb = qc.get("weight_block_size")
    if wb is None:
        return 128
    if len(wb) != 2 or wb[0] != wb[1]:
        raise ValueError(f"weight_block_size {wb} is not square; the FP8 kernels take one block edge")
    return int(wb[0])


def checkpoint_gate_up_interleaved(model_path: str) -> bool:
    """gpt-oss checkpoints interleave the gate and up rows of ``gate_up_proj``."""
    raw = _raw_config(model_path)
    return raw.get("model_type") == "gpt_oss" or "GptOssForCausalLM" in (raw.get("architectures") or [])


# --------------------------------------------------------------------------- safetensors


def safetensors_keys(model_path: str) -> list:
    """Every tensor name of every ``*.safetensors`` shard (headers only, no data)."""
    from safetensors import safe_open

    names = []
    for path in sorted(glob.glob(os.path.join(model_path, "*.safetensors"))):
        with safe_open(path, framework="pt", device="cpu") as f:
            names.extend(f.keys())
    return names


def checkpoint_has_expert_bias(model_path: str) -> bool:
    """Whether the routed experts carry projection biases (any ``experts``
    key ending in ``_bias``: gpt-oss ``gate_up_proj_bias`` / ``down_proj_bias``)."""
    return any("experts" in n.split(".") and n.endswith("_bias") for n in safetensors_keys(model_path))


def iter_safetensors(model_path: str, *, experts_only: bool = True) -> Iterator[Tuple[str, torch.Tensor]]:
    """``(name, tensor)`` over every ``*.safetensors`` shard of ``model_path``
    (file order, then key order), on the CPU; ``experts_only`` keeps the routed
    expert tensors (a key with an ``experts`` segment)."""
    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors files under {model_path!r}")
    for path in files:
        with safe_open(path, framework="pt", device="cpu") as f:
            for name in f.keys():
                if experts_only and "experts" not in name.split("."):
                    continue
                yield name, f.get_tensor(name)


# --------------------------------------------------------------------------- key parsing

_PROJS = ("gate_proj", "up_proj", "down_proj")


def _parse_per_expert_key(key: str, components: tuple, *, mlp_optional: bool) -> Optional[tuple]:
    """``...layers.{L}.[mlp.]experts.{e}.{gate|up|down}_proj.{component}`` ->
    ``(layer, proj, expert, component)``, else None (weight.py:775-812,
    1011-1051, 1397-1441: GPTQ and FP8 keys carry ``mlp``, INT8 keys may not)."""
    parts = key.split(".")
    if len(parts) < 5 or parts[-1] not in components:
        return None
    body = parts[:-1]
    if "experts" not in body:
        return None
    e_pos = body.index("experts")
    has_mlp = e_pos >= 1 and body[e_pos - 1] == "mlp"
    if not has_mlp and not mlp_optional:
        return None
    l_pos = e_pos - 2 if has_mlp else e_pos - 1
    tail = body[e_pos + 1:]
    if l_pos < 0 or len(tail) != 2 or tail[1] not in _PROJS:
        return None
    try:
        return int(body[l_pos]), tail[1], int(tail[0]), parts[-1]
    except ValueError:
        return None


def _parse_fused_key(key: str) -> Optional[tuple]:
    """``...layers.{L}.mlp.experts.{gate_up_proj|down_proj}_{blocks|scales|bias}``
    -> ``(layer, bank, component)`` (weight.py:1231-1273, plus ``_bias``)."""
    parts = key.split(".")
    if "mlp" not in parts or "experts" not in parts:
        return None
    m = parts.index("mlp")
    if m < 1 or m + 1 >= len(parts) or parts[m + 1] != "experts" or len(parts) != m + 3:
        return None
    try:
        layer = int(parts[m - 1])
    except ValueError:
        return None
    token = parts[m + 2]
    for proj, bank in (("gate_up_proj", "gate_up"), ("down_proj", "down")):
        for comp in ("blocks", "scales", "bias"):
            if token == f"{proj}_{comp}":
                return layer, bank, comp
    return None


# --------------------------------------------------------------------------- streaming core


def _stack(rows: list) -> torch.Tensor:
    first = rows[0]
    if any(r.shape != first.shape or r.dtype != first.dtype for r in rows[1:]):
        raise ValueError("per-expert rows of one bank must share one shape and dtype")
    return torch.stack(rows, dim=0).contiguous()


def _stream_per_expert(tensors, config, fmt: str, components: tuple, *, mlp_optional: bool,
                       finalize: Callable) -> Tuple[list, list]:
    """Buffer per-expert components per ``(layer, bank)`` and hand a complete
    bank to ``finalize(per_expert, fuse, layer)`` the moment its last
    component arrives; ``per_expert[e][proj][component]`` -> tensor."""
    L, E = int(config.num_layers), int(config.num_experts)
    buf: Dict[tuple, dict] = {}
    have: Dict[tuple, int] = {}
    done: Dict[tuple, object] = {}
    need = {"gate_up": 2 * len(components) * E, "down": len(components) * E}
    for name, tensor in tensors:
        info = _parse_per_expert_key(name, components, mlp_optional=mlp_optional)
        if info is None:
            raise ValueError(f"Unexpected {fmt} expert weight key: {name}")
        layer, proj, e, comp = info
        bank = "down" if proj == "down_proj" else "gate_up"
        if not 0 <= layer < L:
            raise ValueError(f"Unexpected MoE expert layer {layer}; expected [0, {L})")
        if not 0 <= e < E:
            raise ValueError(f"Unexpected MoE expert id {e} in layer {layer}")
        key = (layer, bank)
        if key in done:
            raise ValueError(f"Layer {layer} {bank!r}: tensor {name!r} arrived after this bank was already "
                             "finalized -- duplicate key or an out-of-order/re-streamed source?")
        slot = buf.setdefault(key, {}).setdefault(e, {}).setdefault(proj, {})
        if comp in slot:
            raise ValueError(f"Duplicate {fmt} component {comp!r} for layer {layer} expert {e} {proj}")
        slot[comp] = tensor
        have[key] = have.get(key, 0) + 1
        if have[key] == need[bank]:
            done[key] = finalize(buf.pop(key), bank == "gate_up", layer)
    missing = [(l, b) for l in range(L) for b in ("gate_up", "down") if (l, b) not in done]
    if missing:
        raise ValueError(f"Missing/incomplete {fmt} MoE expert bank(s): {missing}")
    return [done[(l, "gate_up")] for l in range(L)], [done[(l, "down")] for l in range(L)]


def _fused_pair(per_expert: dict, e: int, layer: int, fmt: str) -> Tuple[dict, dict]:
    gate, up = per_expert[e].get("gate_proj"), per_expert[e].get("up_proj")
    if gate is None or up is None:
        raise ValueError(f"Layer {layer} expert {e}: missing gate_proj/up_proj {fmt} components")
    return gate, up


# --------------------------------------------------------------------------- per format


def stream_moe_expert_sources_gptq(tensors: Iterator[Tuple[str, torch.Tensor]], config) -> Tuple[list, list]:
    """GPTQ per-expert ``qweight/qzeros/scales/g_idx`` -> per-layer
    :class:`GptqExpertBank` pairs (weight.py:814-978): gate and up
    concatenated along N (dim 1), ``g_idx`` checked equal between gate and up
    and across experts, kept once."""

    def finalize(per_expert, fuse, layer):
        rows = []
        for e in range(config.num_experts):
            if fuse:
                gate, up = _fused_pair(per_expert, e, layer, "GPTQ")
                if not torch.equal(gate["g_idx"], up["g_idx"]):
                    raise ValueError(f"Layer {layer} expert {e}: gate_proj/up_proj g_idx mismatch "
                                     "(different group_size/K?)")
                rows.append(tuple(torch.cat([gate[c], up[c]], dim=1) for c in ("qweight", "qzeros", "scales"))
                            + (gate["g_idx"],))
            else:
                d = per_expert[e]["down_proj"]
                rows.append((d["qweight"], d["qzeros"], d["scales"], d["g_idx"]))
        g0 = rows[0][3]
        for e, r in enumerate(rows[1:], start=1):
            if not torch.equal(r[3], g0):
                raise ValueError(f"Layer {layer}: g_idx differs between expert 0 and expert {e}")
        return GptqExpertBank(qweight=_stack([r[0] for r in rows]), qzeros=_stack([r[1] for r in rows]),
                              scales=_stack([r[2] for r in rows]), g_idx=g0)

    return _stream_per_expert(tensors, config, "GPTQ", ("qweight", "qzeros", "scales", "g_idx"), mlp_optional=False,
                              finalize=finalize)


def stream_moe_expert_sources_fp8(tensors: Iterator[Tuple[str, torch.Tensor]], config, *,
                                  block: int = 128) -> Tuple[list, list]:
    """Block-FP8 per-expert ``weight/weight_scale_inv`` -> per-layer
    :class:`Fp8BlockExpertBank` pairs (weight.py:1054-1199): gate and up
    concatenated along N (dim 0), which keeps the fused scale table aligned
    only when the gate's N is a multiple of ``block`` -- checked."""

    def finalize(per_expert, fuse, layer):
        rows = []
        for e in range(config.num_experts):
            if fuse:
                gate, up = _fused_pair(per_expert, e, layer, "block-FP8")
                n_gate = gate["weight"].shape[0]
                if n_gate % block != 0:
                    raise ValueError(f"Layer {layer} expert {e}: gate_proj N={n_gate} is not a multiple of "
                                     f"block={block}; fusing gate_proj+up_proj on the N axis would misalign the "
                                     "fused weight_scale_inv")
                rows.append((torch.cat([gate["weight"], up["weight"]], dim=0),
                             torch.cat([gate["weight_scale_inv"], up["weight_scale_inv"]], dim=0)))
            else:
                d = per_expert[e]["down_proj"]
                rows.append((d["weight"], d["weight_scale_inv"]))
        return Fp8BlockExpertBank(weight=_stack([r[0] for r in rows]), weight_scale_inv=_stack([r[1] for r in rows]))

    return _stream_per_expert(tensors, config, "block-FP8", ("weight", "weight_scale_inv"), mlp_optional=False,
                              finalize=finalize)


def stream_moe_expert_sources_int8(tensors: Iterator[Tuple[str, torch.Tensor]], config) -> Tuple[list, list]:
    """compressed-tensors pack-quantized INT8 per-expert
    ``weight_packed/weight_scale/weight_shape`` -> per-layer
    :class:`Int8ExpertBank` pairs (weight.py:1444-1601): gate and up
    concatenated along N (dim 0); the logical K (``weight_shape[1]``) must
    agree between gate and up and across experts."""

    def k_of(c):
        return int(c["weight_shape"][1].item())

    def finalize(per_expert, fuse, layer):
        rows, k0 = [], None
        for e in range(config.num_experts):
            if fuse:
                gate, up = _fused_pair(per_expert, e, layer, "INT8")
                kg, ku = k_of(gate), k_of(up)
                if kg != ku:
                    raise ValueError(f"Layer {layer} expert {e}: gate_proj K={kg} != up_proj K={ku} "
                                     "(both project the same hidden_size input; a mismatch means a wiring bug)")
                k = kg
                rows.append((torch.cat([gate["weight_packed"], up["weight_packed"]], dim=0),
                             torch.cat([gate["weight_scale"], up["weight_scale"]], dim=0)))
            else:
                d = per_expert[e]["down_proj"]
                k = k_of(d)
                rows.append((d["weight_packed"], d["weight_scale"]))
            if k0 is None:
                k0 = k
            elif k != k0:
                raise ValueError(f"Layer {layer}: expert {e}'s K={k} differs from expert 0's K={k0} "
                                 "(K is an architecture constant, expected identical across every expert)")
        return Int8ExpertBank(weight_packed=_stack([r[0] for r in rows]), weight_scale=_stack([r[1] for r in rows]),
                              k=k0)

    return _stream_per_expert(tensors, config, "INT8", ("weight_packed", "weight_scale", "weight_shape"),
                              mlp_optional=True, finalize=finalize)


def deinterleave_rows(t: torch.Tensor) -> torch.Tensor:
    """``[E, 2I, ...]`` with gate channel i at row 2i and up channel i at row 2i+1
    -> gate rows ``[0, I)`` then up rows ``[I, 2I)``."""
    if t.shape[1] % 2:
        raise ValueError(f"interleaved gate_up has an odd row count {t.shape[1]}")
    return torch.cat([t[:, 0::2], t[:, 1::2]], dim=1).contiguous()


def stream_moe_expert_sources_mxfp4(tensors: Iterator[Tuple[str, torch.Tensor]], config, *,
                                    interleaved_gate_up: bool = False,
                                    expert_bias: Optional[bool] = None) -> Tuple[list, list]:
    """MXFP4 per-layer fused tensors ``{gate_up_proj,down_proj}_{blocks,scales}``
    (one ``[E, ...]`` tensor each, weight.py:1276-1349) and, when present,
    ``_bias`` -> per-layer :class:`MxfpExpertBank` pairs.  ``expert_bias``
    says whether the checkpoint's banks carry biases (``True`` / ``False``,
    e.g. from the shards' key names, :func:`checkpoint_has_expert_bias`): a
    bank is then finalized as soon as its blocks, scales and (if biased) bias
    are in, so one layer at a time is buffered.  ``None`` (unknown): every
    bank is finalized at the end of the stream, since a bias may arrive in a
    later shard than its blocks.  ``interleaved_gate_up``: the gpt-oss row
    order (see :func:`deinterleave_rows`), applied to blocks, scales and
    bias."""
    L = int(config.num_layers)
    buf: Dict[tuple, dict] = {}
    done: Dict[tuple, MxfpExpertBank] = {}
    if expert_bias is None:
        expert_bias = getattr(config, "expert_bias", None)
    biased = bool(expert_bias)

    def finalize(key):
        parts = buf.pop(key)
        blocks, scales, bias = parts["blocks"], parts["scales"], parts.get("bias")
        if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
            raise ValueError(f"Layer {key[0]} {key[1]!r}: MXFP4 blocks/scales must be uint8")
        if blocks.shape[:3] != scales.shape or blocks.shape[-1] != 16:
            raise ValueError(f"Layer {key[0]} {key[1]!r}: blocks {tuple(blocks.shape)} do not match scales "
                             f"{tuple(scales.shape)}")
        if bias is not None and tuple(bias.shape) != tuple(blocks.shape[:2]):
            raise ValueError(f"Layer {key[0]} {key[1]!r}: bias {tuple(bias.shape)} does not match the bank's "
                             f"[E, N] = {tuple(blocks.shape[:2])}")
        if interleaved_gate_up and key[1] == "gate_up":
            blocks, scales = deinterleave_rows(blocks), deinterleave_rows(scales)
            bias = deinterleave_rows(bias[..., None])[..., 0] if bias is not None else None
        done[key] = MxfpExpertBank(blocks=blocks.contiguous(), scales=scales.contiguous(),
                                   bias=bias.contiguous() if bias is not None else None)

    for name, tensor in tensors:
        info = _parse_fused_key(name)
        if info is None:
            raise ValueError(f"Unexpected MXFP4 expert weight key: {name}")
        layer, bank, comp = info
        if not 0 <= layer < L:
            raise ValueError(f"Unexpected MoE expert layer {layer}; expected [0, {L})")
        if tensor.shape[0] != config.num_experts:
            raise ValueError(f"{name}: leading dim {tensor.shape[0]} != num_experts {config.num_experts}")
        key = (layer, bank)
        if comp == "bias" and expert_bias is False:
            raise ValueError(f"{name}: an expert bias in a checkpoint declared without expert biases")
        if key in done:
            raise ValueError(f"Layer {layer} {bank!r}: tensor {name!r} arrived after this bank was already "
                             "finalized -- duplicate key or an out-of-order/re-streamed source?")
        parts = buf.setdefault(key, {})
        if comp in parts:
            raise ValueError(f"Duplicate MXFP4 component {comp!r} for layer {layer} {bank}")
        parts[comp] = tensor
        biased = biased or comp == "bias"
        if expert_bias is not None and "blocks" in parts and "scales" in parts and ("bias" in parts or not biased):
            finalize(key)
    for key in list(buf):
        if "blocks" in buf[key] and "scales" in buf[key]:
            finalize(key)
    missing = [(l, b) for l in range(L) for b in ("gate_up", "down") if (l, b) not in done]
    if missing:
        raise ValueError(f"Missing/incomplete MXFP4 MoE expert bank(s): {missing}")
    if biased and any(done[k].bias is None for k in done):
        raise ValueError("some MXFP4 banks carry a bias and others do not")
    return [done[(l, "gate_up")] for l in range(L)], [done[(l, "down")] for l in range(L)]


# --------------------------------------------------------------------------- entry points


@dataclass(frozen=True)
class MoeCheckpointConfig:
    """What the loader needs of a checkpoint: MoE layers and experts per layer."""

    num_layers: int
    num_experts: int
    hidden_size: int = 0
    moe_intermediate_size: int = 0


def moe_checkpoint_config(model_path: str) -> MoeCheckpointConfig:
    """From ``config.json`` (top level or ``text_config``): ``num_hidden_layers``
    minus ``first_k_dense_replace``, ``num_experts`` (or ``num_local_experts`` /
    ``n_routed_experts``), ``hidden_size``, ``moe_intermediate_size`` (or
    ``intermediate_size``)."""
    raw = _raw_config(model_path)
    c = raw.get("text_config") if isinstance(raw.get("text_config"), dict) else raw
    n_exp = c.get("num_experts") or c.get("num_local_experts") or c.get("n_routed_experts")
    if not n_exp:
        raise ValueError(f"{model_path!r}: config.json names no expert count (not an MoE checkpoint?)")
    layers = int(c["num_hidden_layers"]) - int(c.get("first_k_dense_replace", 0) or 0)
    inter = c.get("moe_intermediate_size") or c.get("intermediate_size") or 0
    return MoeCheckpointConfig(layers, int(n_exp), int(c.get("hidden_size", 0)), int(inter))


def load_moe_expert_sources(model_path: str, config=None) -> Tuple[list, list]:
    """Per-layer packed expert banks ``(gate_up_banks, down_banks)`` of a
    safetensors checkpoint, dispatched on its quantization (weight.py:179-269):
    ``gptq`` -> :class:`GptqExpertBank`, ``fp8`` -> :class:`Fp8BlockExpertBank`,
    ``mxfp4`` -> :class:`MxfpExpertBank` (gpt-oss row order undone),
    compressed-tensors pack-quantized int8 -> :class:`Int8ExpertBank`.
    Anything else raises: the dense bf16 path needs no repacking."""
    config = config if config is not None else moe_checkpoint_config(model_path)
    method = checkpoint_quant_method(model_path)
    src = iter_safetensors(model_path)
    if method == "gptq":
        return stream_moe_expert_sources_gptq(src, config)
    if method == "fp8":
        return stream_moe_expert_sources_fp8(src, config, block=checkpoint_fp8_block(model_path))
    if method == "mxfp4":
        return stream_moe_expert_sources_mxfp4(src, config,
                                               interleaved_gate_up=checkpoint_gate_up_interleaved(model_path),
                                               expert_bias=checkpoint_has_expert_bias(model_path))
    if method == "compressed-tensors" and checkpoint_is_int8_pack_quantized(model_path):
        return stream_moe_expert_sources_int8(src, config)
    raise ValueError(f"{model_path!r}: quantization {method!r} has no packed expert bank in this build "
                     "(gptq, fp8, mxfp4 and compressed-tensors pack-quantized int8 do)")


def bank_format(bank) -> str:
    """The ``OffloadMoeCache`` quant_format of a bank object (loader.py:748-780)."""
    if isinstance(bank, GptqExpertBank):
        return "gptq_int4"
    if isinstance(bank, Fp8BlockExpertBank):
        return "fp8_block"
    if isinstance(bank, MxfpExpertBank):
        return "mxfp4"
    if isinstance(bank, Int8ExpertBank):
        return "int8_channel"
    if isinstance(bank, torch.Tensor):
        return "bf16"
    raise TypeError(f"not an expert bank: {type(bank).__name__}")


def bank_sources(gate_up_banks: list, down_banks: list) -> dict:
    """``{bank name: [per-layer host tensor]}`` in the slot-pool schema of the
    banks' format (offload_cache.py:140-173)."""
    fmt = bank_format(gate_up_banks[0])
    if fmt == "gptq_int4":
        return {"qweight_gate_up": [b.qweight for b in gate_up_banks], "qzeros_gate_up": [b.qzeros for b in gate_up_banks],
                "scales_gate_up": [b.scales for b in gate_up_banks], "qweight_down": [b.qweight for b in down_banks],
                "qzeros_down": [b.qzeros for b in down_banks], "scales_down": [b.scales for b in down_banks]}
    if fmt == "fp8_block":
        return {"weight_gate_up": [b.weight for b in gate_up_banks],
                "scale_gate_up": [b.weight_scale_inv for b in gate_up_banks],
                "weight_down": [b.weight for b in down_banks], "scale_down": [b.weight_scale_inv for b in down_banks]}
    if fmt == "mxfp4":
        src = {"blocks_gate_up": [b.blocks for b in gate_up_banks], "scales_gate_up": [b.scales for b in gate_up_banks],
               "blocks_down": [b.blocks for b in down_banks], "scales_down": [b.scales for b in down_banks]}
        if gate_up_banks[0].bias is not None:  # gpt-oss: per-expert biases ride in the slot like the weights
            src["bias_gate_up"] = [b.bias for b in gate_up_banks]
            src["bias_down"] = [b.bias for b in down_banks]
        return src
    if fmt == "int8_channel":
        return {"weight_packed_gate_up": [b.weight_packed for b in gate_up_banks],
                "weight_scale_gate_up": [b.weight_scale for b in gate_up_banks],
                "weight_packed_down": [b.weight_packed for b in down_banks],
                "weight_scale_down": [b.weight_scale for b in down_banks]}
    return {"gate_up": list(gate_up_banks), "down": list(down_banks)}


def attach_offload_cache(gate_up_banks: list, down_banks: list, *, num_experts: int, device,
                         cache_size: Optional[int] = None, gptq_group_size: Optional[int] = None,
                         fp8_block: int = 128, device_lru: bool = False, decode_only: bool = False):
    """The slot pool over loaded banks (loader.py:693-925): format from the bank
    type, pool size ``num_experts + max(2, layers)`` unless given, the
    attributes :class:`~ftmoe.moe.offload_cache.SlotWeightAccessor` refuses to
    guess (``gptq_group_size`` from the checkpoint, ``int8_k_gate_up`` /
    ``int8_k_down`` from the banks, checked equal across layers), MXFP4
    biases as two more per-slot banks (``bias_gate_up`` / ``bias_down``)."""
    from .moe.offload_cache import OffloadMoeCache

    L = len(gate_up_banks)
    if L == 0 or len(down_banks) != L:
        raise ValueError("gate_up_banks and down_banks must hold one bank per MoE layer")
    fmt = bank_format(gate_up_banks[0])
    if cache_size is None:
        cache_size = num_experts + max(2, L)
    cache = OffloadMoeCache(L, num_experts, cache_size, device, quant_format=fmt, decode_only=decode_only,
                            device_lru=device_lru)
    cache.set_bank_sources(bank_sources(gate_up_banks, down_banks))
    if fmt == "gptq_int4":
        if gptq_group_size is None:
            raise ValueError("attach_offload_cache needs the checkpoint's GPTQ group_size (checkpoint_gptq_group_size)")
        cache.gptq_group_size = int(gptq_group_size)
        cache.set_extra_metadata("g_idx_gate_up", [b.g_idx for b in gate_up_banks])
        cache.set_extra_metadata("g_idx_down", [b.g_idx for b in down_banks])
    elif fmt == "int8_channel":
        ku, kd = {b.k for b in gate_up_banks}, {b.k for b in down_banks}
        if len(ku) != 1 or len(kd) != 1:
            raise ValueError(f"int8_channel: K differs across layers -- gate_up {ku}, down {kd} (K is an "
                             "architecture constant, expected identical across every layer)")
        cache.int8_k_gate_up, cache.int8_k_down = ku.pop(), kd.pop()
    elif fmt == "fp8_block":
        cache.fp8_block_size = int(fp8_block)
    return cache


def moe_layer_from_banks(gate_up, down, *, device, hidden: int, inter: int, topk: int, num_experts: int,
                         gate_w: Optional[torch.Tensor] = None, gate_b: Optional[torch.Tensor] = None,
                         shared: Optional[dict] = None, route_mode: str = "softmax_topk", act: str = "silu",
                         group: Optional[int] = None, swiglu_alpha: float = 1.702, swiglu_limit: float = 7.0):
    """One layer's loaded banks moved to ``device`` as a
    :class:`~ftmoe.layer.MoeLayer` whose experts live in HBM (the in-VRAM
    forward, python/freetoken/models/qwen3_5_moe/__init__.py:1331-1373, as one
    grouped call).  ``group``: the GPTQ group size or FP8 block edge (the
    INT8 group comes from the scales' shape)."""
    from .banks import proj_from_bank
    from .layer import MoeLayer

    fmt = bank_format(gate_up)
    src = bank_sources([gate_up], [down])
    bank = {k: v[0].to(device) for k, v in src.items()}
    b13 = b2 = None
    if fmt == "mxfp4":
        group = 32
        b13 = gate_up.bias.to(device, torch.bfloat16) if gate_up.bias is not None else None
        b2 = down.bias.to(device, torch.bfloat16) if down.bias is not None else None
    elif fmt == "fp8_block" and group is None:
        group = 128
    elif fmt == "gptq_int4" and group is None:
        raise ValueError("moe_layer_from_banks needs the GPTQ group size")
    ku, kd = (gate_up.k, down.k) if fmt == "int8_channel" else (hidden, inter)
    w13 = proj_from_bank(fmt, bank, which="gate_up", N=2 * inter, K=ku, group=group, bias=b13)
    w2 = proj_from_bank(fmt, bank, which="down", N=hidden, K=kd, group=group, bias=b2)
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    return MoeLayer(w13=w13, w2=w2, num_experts=num_experts, hidden=hidden, inter=inter, topk=topk,
                    gate_w=dev(gate_w), gate_b=dev(gate_b),
                    shared={k: v.to(device) for k, v in shared.items()} if shared else None,
                    route_mode=route_mode, act=act, swiglu_alpha=swiglu_alpha, swiglu_limit=swiglu_limit)


__all__ = [
    "GptqExpertBank", "Fp8BlockExpertBank", "MxfpExpertBank", "Int8ExpertBank", "MoeCheckpointConfig",
    "checkpoint_quant_method", "checkpoint_is_int8_pack_quantized", "checkpoint_int8_pack_quantized_group_size",
    "checkpoint_gptq_group_size", "checkpoint_fp8_block", "checkpoint_gate_up_interleaved", "iter_safetensors",
    "safetensors_keys", "checkpoint_has_expert_bias",
    "stream_moe_expert_sources_gptq", "stream_moe_expert_sources_fp8", "stream_moe_expert_sources_int8",
    "stream_moe_expert_sources_mxfp4", "deinterleave_rows", "moe_checkpoint_config", "load_moe_expert_sources",
    "bank_format", "bank_sources", "attach_offload_cache", "moe_layer_from_banks",
]
