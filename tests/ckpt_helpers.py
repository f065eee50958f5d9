"""Fabricated safetensors checkpoints in the reference's key spellings, written
from a synthetic layer's banks (what a quantized HF checkpoint of that
format holds), for the loader tests."""
from __future__ import annotations

import json
import os

import torch


def _split_gate_up(t: torch.Tensor, dim: int, n_gate: int):
    return t.narrow(dim, 0, n_gate), t.narrow(dim, n_gate, t.shape[dim] - n_gate)


def interleave_rows(t: torch.Tensor) -> torch.Tensor:
    """[E, 2I, ...] gate-then-up -> gpt-oss order (gate channel i at row 2i, up at 2i + 1)."""
    I = t.shape[1] // 2
    out = torch.empty_like(t)
    out[:, 0::2], out[:, 1::2] = t[:, :I], t[:, I:]
    return out


def expert_tensors(fmt: str, syn, layer: int) -> dict:
    """{key: tensor} of one layer's routed experts, per the format's checkpoint layout."""
    cfg, b = syn.cfg, syn.bank
    I, H = cfg.I, cfg.H
    out = {}
    if fmt == "mxfp4":
        pre = f"model.layers.{layer}.mlp.experts."
        out[pre + "gate_up_proj_blocks"] = interleave_rows(b["blocks_gate_up"])
        out[pre + "gate_up_proj_scales"] = interleave_rows(b["scales_gate_up"])
        out[pre + "down_proj_blocks"] = b["blocks_down"].clone()
        out[pre + "down_proj_scales"] = b["scales_down"].clone()
        if syn.bias13 is not None:
            out[pre + "gate_up_proj_bias"] = interleave_rows(syn.bias13[..., None])[..., 0].contiguous()
            out[pre + "down_proj_bias"] = syn.bias2.clone()
        return out
    for e in range(cfg.E):
        if fmt == "gptq_int4":
            pre = f"model.layers.{layer}.mlp.experts.{e}."
            g_idx = torch.arange(H, dtype=torch.int32) // cfg.group
            qg, qu = _split_gate_up(b["qweight_gate_up"][e], 1, I)
            zg, zu = _split_gate_up(b["qzeros_gate_up"][e], 1, I // 8)
            sg, su = _split_gate_up(b["scales_gate_up"][e], 1, I)
            for proj, (q, z, s) in (("gate_proj", (qg, zg, sg)), ("up_proj", (qu, zu, su))):
                out[pre + proj + ".qweight"], out[pre + proj + ".qzeros"] = q.contiguous(), z.contiguous()
                out[pre + proj + ".scales"], out[pre + proj + ".g_idx"] = s.contiguous(), g_idx.clone()
            out[pre + "down_proj.qweight"] = b["qweight_down"][e].clone()
            out[pre + "down_proj.qzeros"] = b["qzeros_down"][e].clone()
            out[pre + "down_proj.scales"] = b["scales_down"][e].clone()
            out[pre + "down_proj.g_idx"] = torch.arange(I, dtype=torch.int32) // cfg.group
        elif fmt == "fp8_block":
            pre = f"model.layers.{layer}.mlp.experts.{e}."
            wg, wu = _split_gate_up(b["weight_gate_up"][e], 0, I)
            sg, su = _split_gate_up(b["scale_gate_up"][e], 0, I // cfg.group)
            for proj, (w, s) in (("gate_proj", (wg, sg)), ("up_proj", (wu, su))):
                out[pre + proj + ".weight"], out[pre + proj + ".weight_scale_inv"] = w.contiguous(), s.contiguous()
            out[pre + "down_proj.weight"] = b["weight_down"][e].clone()
            out[pre + "down_proj.weight_scale_inv"] = b["scale_down"][e].clone()
        elif fmt == "int8_channel":
            pre = f"model.language_model.layers.{layer}.experts.{e}."  # the no-mlp spelling of real INT8 checkpoints
            wg, wu = _split_gate_up(b["weight_packed_gate_up"][e], 0, I)
            sg, su = _split_gate_up(b["weight_scale_gate_up"][e], 0, I)
            for proj, (w, s) in (("gate_proj", (wg, sg)), ("up_proj", (wu, su))):
                out[pre + proj + ".weight_packed"], out[pre + proj + ".weight_scale"] = w.contiguous(), s.contiguous()
                out[pre + proj + ".weight_shape"] = torch.tensor([I, H], dtype=torch.int64)
            out[pre + "down_proj.weight_packed"] = b["weight_packed_down"][e].clone()
            out[pre + "down_proj.weight_scale"] = b["weight_scale_down"][e].clone()
            out[pre + "down_proj.weight_shape"] = torch.tensor([H, I], dtype=torch.int64)
        else:
            raise ValueError(fmt)
    return out


def quant_config(fmt: str, cfg) -> dict:
    if fmt == "gptq_int4":
        return {"quant_method": "gptq", "bits": 4, "group_size": cfg.group, "desc_act": False, "sym": True}
    if fmt == "fp8_block":
        return {"quant_method": "fp8", "fmt": "e4m3", "activation_scheme": "dynamic",
                "weight_block_size": [cfg.group, cfg.group]}
    if fmt == "mxfp4":
        return {"quant_method": "mxfp4"}
    if fmt == "int8_channel":
        return {"quant_method": "compressed-tensors", "format": "pack-quantized",
                "config_groups": {"group_0": {"format": "pack-quantized", "targets": ["Linear"],
                                              "weights": {"num_bits": 8, "type": "int", "symmetric": True,
                                                          "strategy": "channel", "group_size": None}}}}
    raise ValueError(fmt)


def write_checkpoint(path, fmt: str, syns: list, *, shards: int = 2) -> None:
    """config.json + the layers' expert tensors spread over ``shards`` files
    (keys dealt round-robin, so one layer's components span several shards)."""
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    cfg = syns[0].cfg
    keys = {}
    for layer, syn in enumerate(syns):
        keys.update(expert_tensors(fmt, syn, layer))
    names = list(keys)
    for s in range(shards):
        part = {n: keys[n].contiguous() for n in names[s::shards]}
        save_file(part, os.path.join(path, f"model-{s + 1:05d}-of-{shards:05d}.safetensors"))
    conf = {"architectures": ["GptOssForCausalLM" if fmt == "mxfp4" else "Qwen3MoeForCausalLM"],
            "model_type": "gpt_oss" if fmt == "mxfp4" else "qwen3_moe", "num_hidden_layers": len(syns),
            "hidden_size": cfg.H, "moe_intermediate_size": cfg.I, "quantization_config": quant_config(fmt, cfg)}
    conf["num_local_experts" if fmt == "mxfp4" else "num_experts"] = cfg.E
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(conf, f)
