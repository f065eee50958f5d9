"""GPU: banks loaded from fabricated safetensors checkpoints (ftmoe.loader) run
the layer to oracle parity -- in HBM (moe_layer_from_banks) for every format,
gpt-oss's interleaved and biased MXFP4 gate_up included, and through the slot
pool the loader wires (attach_offload_cache + moe_offload_forward)."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ckpt_helpers import write_checkpoint
from ftm_helpers import assert_close, np_, oracle_spec, to_f32

from ftmoe import loader as LD
from ftmoe import synthetic as S
from ftmoe.moe.offload_cache import moe_offload_forward

pytestmark = pytest.mark.gpu

FMT_OF = {"c1_int8": "int8_channel", "c2_gptq": "gptq_int4", "c3_fp8": "fp8_block", "c4_mxfp4": "mxfp4"}


@pytest.mark.parametrize("name", list(FMT_OF))
def test_loaded_banks_match_oracle(gpu, tmp_path, name):
    cfg = S.SMALL[name]
    syns = [S.generate(cfg, T=9, seed=300 + l) for l in range(2)]
    write_checkpoint(tmp_path, FMT_OF[name], syns)
    gu, dn = LD.load_moe_expert_sources(str(tmp_path))
    syn = syns[1]
    group = LD.checkpoint_gptq_group_size(str(tmp_path)) if name == "c2_gptq" else cfg.group
    layer = LD.moe_layer_from_banks(gu[1], dn[1], device=gpu, hidden=cfg.H, inter=cfg.I, topk=cfg.k,
                                    num_experts=cfg.E, gate_w=syn.gate_w, gate_b=syn.gate_b, shared=syn.shared,
                                    route_mode=cfg.route_mode, act=cfg.act, group=group)
    out, ids, _, _ = layer.forward(syn.x.to(gpu), return_routing=True)
    ref = O.layer_reference(oracle_spec(syn), np_(syn.x))
    np.testing.assert_array_equal(ids.cpu().numpy(), ref["ids"])
    assert_close(to_f32(out), ref["out"], what=f"{name} layer from loaded banks")


def test_loaded_fp8_banks_through_the_slot_pool(gpu, tmp_path):
    cfg = S.SMALL["c3_fp8"]
    syns = [S.generate(cfg, T=6, seed=310 + l) for l in range(2)]
    write_checkpoint(tmp_path, "fp8_block", syns)
    gu, dn = LD.load_moe_expert_sources(str(tmp_path))
    cache = LD.attach_offload_cache(gu, dn, num_experts=cfg.E, device=gpu, cache_size=12, decode_only=True,
                                    fp8_block=LD.checkpoint_fp8_block(str(tmp_path)))
    rng = np.random.RandomState(3)
    for step in range(4):
        l = step % 2
        syn = syns[l]
        ids = np.stack([rng.choice(cfg.E, cfg.k, replace=False) for _ in range(6)]).astype(np.int32)
        w = O.round_bf16(rng.rand(6, cfg.k).astype(np.float32))
        out = moe_offload_forward(syn.x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), cache, l,
                                  intermediate=cfg.I, shared={k: v.to(gpu) for k, v in syn.shared.items()})
        ref = O.layer_reference(oracle_spec(syn), np_(syn.x), ids=ids, w=w)
        assert_close(to_f32(out), ref["out"], what=f"slot-pool step {step}")
    cache.check_status()
