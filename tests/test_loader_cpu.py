"""The checkpoint loader (ftmoe.loader) on fabricated safetensors checkpoints,
CPU only, in the manner of the reference's tests/test_weight_{gptq,fp8,int8,
mxfp4}_banks.py: format detection from config.json, every format's banks
streamed back bit for bit from the per-expert (GPTQ/FP8/INT8) or per-layer
fused (MXFP4) key spellings, gate rows first, gpt-oss's interleaved and biased
gate_up undone, the reference's known GPTQ fixture value, the loud errors, and
the slot-pool wiring."""
import json
from dataclasses import replace
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import ftm_oracle as O
from ckpt_helpers import expert_tensors, interleave_rows, write_checkpoint

from ftmoe import loader as LD
from ftmoe import synthetic as S

FMT_OF = {"c1_int8": "int8_channel", "c2_gptq": "gptq_int4", "c3_fp8": "fp8_block", "c4_mxfp4": "mxfp4"}


def _syns(name, layers=2):
    cfg = replace(S.SMALL[name], E=4)
    return [S.generate(cfg, T=3, seed=100 + l) for l in range(layers)]


@pytest.mark.parametrize("name", list(FMT_OF))
def test_checkpoint_banks_round_trip(tmp_path, name):
    """Loading the fabricated checkpoint gives back exactly the banks it was
    written from (gate rows first), through the format detected from
    config.json, with the keys of one layer spread over two shards."""
    fmt = FMT_OF[name]
    syns = _syns(name)
    write_checkpoint(tmp_path, fmt, syns)
    assert LD.checkpoint_quant_method(str(tmp_path)) == {"gptq_int4": "gptq", "fp8_block": "fp8", "mxfp4": "mxfp4",
                                                         "int8_channel": "compressed-tensors"}[fmt]
    gu, dn = LD.load_moe_expert_sources(str(tmp_path))
    assert len(gu) == len(dn) == 2
    for layer, syn in enumerate(syns):
        src = LD.bank_sources([gu[layer]], [dn[layer]])
        bias = {"bias_gate_up": syn.bias13, "bias_down": syn.bias2} if fmt == "mxfp4" else {}
        assert set(src) == set(syn.bank) | set(bias)
        for k, v in bias.items():
            assert torch.equal(src.pop(k)[0], v)
        for k, v in src.items():
            assert v[0].dtype == syn.bank[k].dtype and torch.equal(v[0].view(torch.uint8), syn.bank[k].view(torch.uint8)), k
        if fmt == "mxfp4":
            assert torch.equal(gu[layer].bias, syn.bias13) and torch.equal(dn[layer].bias, syn.bias2)
        if fmt == "int8_channel":
            assert gu[layer].k == syn.cfg.H and dn[layer].k == syn.cfg.I
        if fmt == "gptq_int4":
            assert torch.equal(gu[layer].g_idx, torch.arange(syn.cfg.H, dtype=torch.int32) // syn.cfg.group)


def test_gptq_known_fixture_value():
    """The reference's own fixture (tests/test_weight_gptq_banks.py:90-111):
    weight code 5, zero code 7 (+1), scale 0.5 dequantize to -1.5 everywhere,
    for both halves of the fused gate_up bank and for down."""
    k, n, g = 16, 8, 8

    def pack(c):
        w = sum(c << (4 * i) for i in range(8))
        return w - (1 << 32) if w >= 1 << 31 else w

    def proj():
        return {"qweight": torch.full((k // 8, n), pack(5), dtype=torch.int32),
                "qzeros": torch.full((k // g, n // 8), pack(7), dtype=torch.int32),
                "scales": torch.full((k // g, n), 0.5, dtype=torch.float16),
                "g_idx": torch.arange(k, dtype=torch.int32) // g}

    def stream():
        for e in range(2):
            for p in ("gate_proj", "up_proj", "down_proj"):
                for c, t in proj().items():
                    yield f"model.layers.0.mlp.experts.{e}.{p}.{c}", t

    gu, dn = LD.stream_moe_expert_sources_gptq(stream(), SimpleNamespace(num_layers=1, num_experts=2))
    for e in range(2):
        d = O.dequantize_gptq_int4(dn[0].qweight[e].numpy(), dn[0].qzeros[e].numpy(), dn[0].scales[e].float().numpy(), g)
        assert np.all(d == -1.5) and d.shape == (k, n)
        f = O.dequantize_gptq_int4(gu[0].qweight[e].numpy(), gu[0].qzeros[e].numpy(), gu[0].scales[e].float().numpy(), g)
        assert np.all(f == -1.5) and f.shape == (k, 2 * n)


def test_gate_up_concat_keeps_each_half(tmp_path):
    """Gate and up halves quantized independently stay in their own rows:
    gate's rows [0, I), up's [I, 2I) (FP8: dim 0; GPTQ: the N axis, dim 1)."""
    syns = _syns("c3_fp8", layers=1)
    t = expert_tensors("fp8_block", syns[0], 0)
    gu, _ = LD.stream_moe_expert_sources_fp8(iter(t.items()), SimpleNamespace(num_layers=1, num_experts=4))
    I = syns[0].cfg.I
    for e in range(4):
        assert torch.equal(gu[0].weight[e, :I].view(torch.uint8),
                           t[f"model.layers.0.mlp.experts.{e}.gate_proj.weight"].view(torch.uint8))
        assert torch.equal(gu[0].weight[e, I:].view(torch.uint8),
                           t[f"model.layers.0.mlp.experts.{e}.up_proj.weight"].view(torch.uint8))


def test_gpt_oss_interleaved_gate_up_is_split():
    """gpt-oss rows: gate channel i at row 2i, up channel i at 2i + 1; the
    bank holds gate rows then up rows (blocks, scales and bias alike)."""
    x = torch.arange(2 * 6 * 3, dtype=torch.int32).reshape(2, 6, 3)
    y = LD.deinterleave_rows(x)
    assert torch.equal(y[:, :3], x[:, 0::2]) and torch.equal(y[:, 3:], x[:, 1::2])
    assert torch.equal(LD.deinterleave_rows(interleave_rows(x)), x)


def _fp8_stream(syn, layer=0):
    return list(expert_tensors("fp8_block", syn, layer).items())


def test_stream_errors_are_loud():
    syn = _syns("c3_fp8", layers=1)[0]
    cfg = SimpleNamespace(num_layers=1, num_experts=4)
    items = _fp8_stream(syn)
    with pytest.raises(ValueError, match="Unexpected block-FP8 expert weight key"):
        LD.stream_moe_expert_sources_fp8(iter(items + [("model.layers.0.mlp.gate.weight", torch.zeros(1))]), cfg)
    with pytest.raises(ValueError, match="Duplicate"):
        LD.stream_moe_expert_sources_fp8(iter(items[:1] + items), cfg)
    with pytest.raises(ValueError, match="already finalized"):
        LD.stream_moe_expert_sources_fp8(iter(items + items[:1]), cfg)
    with pytest.raises(ValueError, match="Missing/incomplete"):
        LD.stream_moe_expert_sources_fp8(iter(items[:-1]), cfg)
    with pytest.raises(ValueError, match="expert id 7"):
        LD.stream_moe_expert_sources_fp8(iter([("model.layers.0.mlp.experts.7.down_proj.weight", torch.zeros(1))]), cfg)
    with pytest.raises(ValueError, match="layer 3"):
        LD.stream_moe_expert_sources_fp8(iter([("model.layers.3.mlp.experts.0.down_proj.weight", torch.zeros(1))]), cfg)
    # gate N not a multiple of the block: the fused scale table would misalign
    with pytest.raises(ValueError, match="not a multiple of block"):
        LD.stream_moe_expert_sources_fp8(iter(items), cfg, block=96)


def test_int8_and_gptq_consistency_errors():
    syn = _syns("c1_int8", layers=1)[0]
    cfg = SimpleNamespace(num_layers=1, num_experts=4)
    t = expert_tensors("int8_channel", syn, 0)
    key = next(k for k in t if k.endswith("experts.0.up_proj.weight_shape"))
    t[key] = torch.tensor([syn.cfg.I, syn.cfg.H + 4], dtype=torch.int64)
    with pytest.raises(ValueError, match="gate_proj K=.* != up_proj K"):
        LD.stream_moe_expert_sources_int8(iter(t.items()), cfg)
    sg = _syns("c2_gptq", layers=1)[0]
    t = expert_tensors("gptq_int4", sg, 0)
    key = next(k for k in t if k.endswith("experts.1.up_proj.g_idx"))
    t[key] = torch.zeros_like(t[key])
    with pytest.raises(ValueError, match="g_idx mismatch"):
        LD.stream_moe_expert_sources_gptq(iter(t.items()), cfg)


def test_format_detection_and_group_sizes(tmp_path):
    syns = _syns("c1_int8", layers=1)
    write_checkpoint(tmp_path, "int8_channel", syns)
    p = str(tmp_path)
    assert LD.checkpoint_is_int8_pack_quantized(p) and LD.checkpoint_int8_pack_quantized_group_size(p) is None
    c = LD.moe_checkpoint_config(p)
    assert (c.num_layers, c.num_experts, c.hidden_size, c.moe_intermediate_size) == (1, 4, syns[0].cfg.H, syns[0].cfg.I)
    q = tmp_path / "gptq"
    write_checkpoint(q, "gptq_int4", _syns("c2_gptq", layers=1))
    assert LD.checkpoint_gptq_group_size(str(q)) == 128 and not LD.checkpoint_is_int8_pack_quantized(str(q))
    with pytest.raises(ValueError, match="group_size"):
        LD.checkpoint_gptq_group_size(p)
    m = tmp_path / "mx"
    write_checkpoint(m, "mxfp4", _syns("c4_mxfp4", layers=1))
    assert LD.checkpoint_gate_up_interleaved(str(m)) and not LD.checkpoint_gate_up_interleaved(p)


@pytest.mark.parametrize("name", list(FMT_OF))
def test_attach_offload_cache_wires_the_slot_api(tmp_path, name):
    fmt = FMT_OF[name]
    syns = _syns(name)
    write_checkpoint(tmp_path, fmt, syns)
    gu, dn = LD.load_moe_expert_sources(str(tmp_path))
    gs = LD.checkpoint_gptq_group_size(str(tmp_path)) if fmt == "gptq_int4" else None
    c = LD.attach_offload_cache(gu, dn, num_experts=4, device="cpu", gptq_group_size=gs)
    assert c.quant_format == fmt and c.cache_size == 4 + 2
    assert set(c.bank_schema) == set(syns[0].bank) | ({"bias_gate_up", "bias_down"} if fmt == "mxfp4" else set())
    if fmt == "gptq_int4":
        assert c.gptq_group_size == 128 and len(c.get_extra_metadata("g_idx_down", 1)) == syns[0].cfg.I
    if fmt == "int8_channel":
        assert (c.int8_k_gate_up, c.int8_k_down) == (syns[0].cfg.H, syns[0].cfg.I)
    if fmt == "mxfp4":
        assert torch.equal(c.bank_sources["bias_gate_up"][1], syns[1].bias13)
        assert c.bank_caches["bias_down"].shape == (c.cache_size, syns[0].cfg.H)
    if fmt == "gptq_int4":
        with pytest.raises(ValueError, match="group_size"):
            LD.attach_offload_cache(gu, dn, num_experts=4, device="cpu")


def test_mxfp4_biases_in_a_later_shard(tmp_path):
    """gpt-oss expert biases stored in a shard after every block and scale:
    the loader learns from the shards' key names that the checkpoint is
    biased and waits for each bank's bias (before, a bank was finalized as
    soon as its blocks and scales arrived, and the late bias was refused as
    a re-streamed key).  An unknown bias state defers every bank to the end
    of the stream; a declared bias-free checkpoint refuses a bias."""
    from safetensors.torch import save_file

    from ckpt_helpers import expert_tensors, quant_config

    syns = _syns("c4_mxfp4")
    keys = {}
    for layer, syn in enumerate(syns):
        keys.update(expert_tensors("mxfp4", syn, layer))
    weights = {n: t.contiguous() for n, t in keys.items() if not n.endswith("_bias")}
    biases = {n: t.contiguous() for n, t in keys.items() if n.endswith("_bias")}
    assert biases
    save_file(weights, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(biases, str(tmp_path / "model-00002-of-00002.safetensors"))
    cfg = syns[0].cfg
    conf = {"architectures": ["GptOssForCausalLM"], "model_type": "gpt_oss", "num_hidden_layers": len(syns),
            "hidden_size": cfg.H, "moe_intermediate_size": cfg.I, "num_local_experts": cfg.E,
            "quantization_config": quant_config("mxfp4", cfg)}
    (tmp_path / "config.json").write_text(json.dumps(conf))
    assert LD.checkpoint_has_expert_bias(str(tmp_path))
    gu, dn = LD.load_moe_expert_sources(str(tmp_path))
    for layer, syn in enumerate(syns):
        assert torch.equal(gu[layer].bias, syn.bias13) and torch.equal(dn[layer].bias, syn.bias2)
        assert torch.equal(gu[layer].blocks, syn.bank["blocks_gate_up"])
    config = LD.moe_checkpoint_config(str(tmp_path))
    src = lambda: LD.iter_safetensors(str(tmp_path))  # noqa: E731
    gu2, dn2 = LD.stream_moe_expert_sources_mxfp4(src(), config, interleaved_gate_up=True)  # bias state unknown
    assert all(torch.equal(a.bias, b.bias) for a, b in zip(gu + dn, gu2 + dn2))
    with pytest.raises(ValueError, match="declared without expert biases"):
        LD.stream_moe_expert_sources_mxfp4(src(), config, interleaved_gate_up=True, expert_bias=False)
