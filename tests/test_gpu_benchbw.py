"""GPU: the calibration command (ftmoe.moe.benchbw.main, ``ft bench bw``) on
the real box at a small shape -- the profile it writes is read back by the
reader, its numbers are positive and its fetch fraction is the reader's --
and an offload MoeBlock stepping through the hybrid split with the fraction
from that profile ("auto") matches the oracle."""
import json

import pytest
import torch

import ftm_oracle as O
from ftm_helpers import assert_close, np_, oracle_spec, to_f32

from ftmoe import synthetic as S
from ftmoe.engine import MoeBlock
from ftmoe.moe import bench_profile as BP
from ftmoe.moe import benchbw as BW
from ftmoe.moe.offload_cache import OffloadMoeCache

pytestmark = pytest.mark.gpu


def test_benchbw_writes_a_profile_the_reader_uses(gpu, tmp_path, monkeypatch):
    out = tmp_path / "prof.json"
    rc = BW.main(["--dtype", "fp8_block,gptq_int4", "--experts", "16", "--intermediate", "256", "--hidden", "512",
                  "--repeats", "3", "--out", str(out), "--threads", "4"])
    assert rc == 0
    prof = json.loads(out.read_text())
    name, uuid = BP.gpu_identity()
    assert prof["gpu"]["name"] == name and name
    for fmt in ("fp8_block", "gptq_int4"):
        e = prof["dtype_kernels"][fmt]
        print(fmt, e, flush=True)
        for k in ("cpu_moe_gbs", "pcie_gather_gbs", "cpu_moe_overlap_gbs", "pcie_gather_overlap_gbs", "hbm_copy_gbs"):
            assert e[k] > 0, k
        assert prof["dtypes"][fmt] == e["recommended"] in ("hybrid", "offload")
        assert 0 < e["fetch_fraction"] < 1
        monkeypatch.setenv(BP.ENV_PROFILE_PATH, str(out))
        assert BP.load_backend_recommendation(fmt) == e["recommended"]
        f = BP.load_hybrid_fetch_fraction(fmt)
        assert f == pytest.approx(e["pcie_gather_overlap_gbs"] /
                                  (e["pcie_gather_overlap_gbs"] + e["cpu_moe_overlap_gbs"]), rel=1e-6)
        assert f == pytest.approx(e["fetch_fraction"], abs=1e-4)


def test_offload_block_with_auto_fraction_steps_through_the_split(gpu, tmp_path, monkeypatch):
    cfg = S.SMALL["c3_fp8"]
    syn = S.generate(cfg, T=6, seed=410)
    name, uuid = BP.gpu_identity()
    prof = {"gpu": {"name": name, "uuid": uuid}, "dtypes": {"fp8_block": "hybrid"},
            "dtype_kernels": {"fp8_block": {"cpu_moe_overlap_gbs": 30.0, "pcie_gather_overlap_gbs": 10.0}}}
    p = tmp_path / "prof.json"
    p.write_text(json.dumps(prof))
    monkeypatch.setenv(BP.ENV_PROFILE_PATH, str(p))
    c = OffloadMoeCache(1, cfg.E, 16, gpu, quant_format="fp8_block", decode_only=True)
    c.set_bank_sources({b: [syn.bank[b]] for b in c.bank_schema})
    sh = {k: v.to(gpu) for k, v in syn.shared.items()}
    Is = cfg.shared_inter
    block = MoeBlock(gate=syn.gate_w.to(gpu), top_k=cfg.k, intermediate=cfg.I,
                     shared=(sh["w13"][:Is], sh["w13"][Is:], sh["w2"], sh["gate"]), cache=c, layer_id=0,
                     hybrid_fetch_fraction="auto")
    assert block.hybrid_fetch_fraction == pytest.approx(0.25)
    spec = oracle_spec(syn)
    for step in range(3):
        x = syn.x[2 * step:2 * step + 2]
        out = block(x.to(gpu))
        ref = O.layer_reference(spec, np_(x))
        assert_close(to_f32(out), ref["out"], what=f"hybrid block step {step}")
