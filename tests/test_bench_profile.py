"""The calibration profile: the reader (ftmoe.moe.bench_profile, restating
tests/test_moe_hybrid_profile.py:1-265 of the reference) and the writer's
host-side parts (ftmoe.moe.benchbw: verdict, fetch fraction, packed banks and
their bytes, the CPU half's bandwidth, the workload resolution, no-GPU exit)."""
import json
import os

import pytest

from ftmoe.moe import bench_profile as BP
from ftmoe.moe import benchbw as BW
from ftmoe import synthetic as S


def _hybrid_profile() -> dict:
    """CPU 3x the PCIe gather standalone (hybrid); overlapped 20 : 8 -> f = 8 / 28."""
    return {"gpu": {"name": "Test GPU", "uuid": "uuid-0"}, "dtypes": {"bf16": "hybrid"},
            "dtype_kernels": {"bf16": {"cpu_moe_gbs": 30.0, "pcie_gather_gbs": 10.0,
                                       "cpu_moe_overlap_gbs": 20.0, "pcie_gather_overlap_gbs": 8.0}}}


def _offload_profile() -> dict:
    return {"gpu": {"name": "Test GPU", "uuid": "uuid-0"}, "dtypes": {"bf16": "offload"},
            "dtype_kernels": {"bf16": {"cpu_moe_gbs": 12.0, "pcie_gather_gbs": 10.0}}}


def _write(tmp_path, prof) -> str:
    p = str(tmp_path / "prof.json")
    with open(p, "w") as f:
        json.dump(prof, f)
    return p


@pytest.fixture(autouse=True)
def _no_env(monkeypatch):
    monkeypatch.delenv(BP.ENV_PROFILE_PATH, raising=False)


def test_profile_path_keyed_per_gpu_uuid(tmp_path, monkeypatch):
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    assert BP.default_profile_path("abcd-1234") == str(tmp_path / "freetoken" / "benchbw" / "abcd-1234.json")
    assert BP.default_profile_path() == str(tmp_path / "freetoken" / "benchbw.json")


def test_latest_profile_path(tmp_path, monkeypatch):
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    (tmp_path / "freetoken").mkdir()
    assert BP.latest_profile_path() is None
    legacy = tmp_path / "freetoken" / "benchbw.json"
    legacy.write_text("{}")
    assert BP.latest_profile_path() == str(legacy)
    per = tmp_path / "freetoken" / "benchbw"
    per.mkdir()
    (per / "a.json").write_text("{}")
    os.utime(per / "a.json", (1, 1))
    (per / "b.json").write_text("{}")
    assert BP.latest_profile_path() == str(per / "b.json")  # the newest per-device file


def test_recommendations(tmp_path):
    assert BP.load_backend_recommendation("bf16", path=_write(tmp_path, _hybrid_profile())) == "hybrid"
    assert BP.load_backend_recommendation("bf16", path=_write(tmp_path, _offload_profile())) == "offload"
    assert BP.load_backend_recommendation("fp8_block", path=_write(tmp_path, _hybrid_profile())) is None


def test_mixed_workload_verdict_is_offload(tmp_path):
    prof = {"gpu": {"name": "Test GPU"}, "workloads": {
        "a": {"kernels": {"bf16": {"recommended": "hybrid"}}},
        "b": {"kernels": {"bf16": {"recommended": "offload"}}}}}
    assert BP.load_backend_recommendation("bf16", path=_write(tmp_path, prof)) == "offload"
    prof["workloads"]["b"]["kernels"]["bf16"]["recommended"] = "hybrid"
    assert BP.load_backend_recommendation("bf16", path=_write(tmp_path, prof)) == "hybrid"


def test_device_mismatch_and_unreadable_profiles_are_ignored(tmp_path):
    prof = _hybrid_profile()
    prof["gpu"]["name"] = "Another GPU"
    p = _write(tmp_path, prof)
    assert BP.load_backend_recommendation("bf16", gpu_name="Test GPU", path=p) is None
    assert BP.load_backend_recommendation("bf16", xpu_name="Test GPU", path=p) is None  # the reference's keyword
    assert BP.load_backend_recommendation("bf16", gpu_name="Another GPU", path=p) == "hybrid"
    bad = tmp_path / "bad.json"
    bad.write_text("not json {")
    assert BP.load_backend_recommendation("bf16", path=str(bad)) is None


def test_reference_xpu_block_and_mxfp4_triton_key_are_read(tmp_path):
    prof = {"xpu": {"name": "Test GPU"}, "dtypes": {"mxfp4_triton": "hybrid"},
            "dtype_kernels": {"mxfp4_triton": {"cpu_moe_overlap_gbs": 30.0, "pcie_gather_overlap_gbs": 10.0}}}
    p = _write(tmp_path, prof)
    assert BP.load_backend_recommendation("mxfp4", gpu_name="Test GPU", path=p) == "hybrid"
    assert BP.load_hybrid_fetch_fraction("mxfp4", path=p) == pytest.approx(0.25)


def test_fetch_fraction(tmp_path):
    p = _write(tmp_path, _hybrid_profile())
    assert BP.load_hybrid_fetch_fraction("bf16", gpu_uuid="uuid-0", path=p) == pytest.approx(8 / 28, abs=1e-12)
    prof = _hybrid_profile()
    del prof["dtype_kernels"]["bf16"]["cpu_moe_overlap_gbs"], prof["dtype_kernels"]["bf16"]["pcie_gather_overlap_gbs"]
    # the reference reader's standalone fallback is pcie / cpu (its test pins 10 / 30)
    assert BP.load_hybrid_fetch_fraction("bf16", path=_write(tmp_path, prof)) == pytest.approx(10 / 30, abs=1e-12)
    zero = {"gpu": {"name": "Test GPU"}, "dtype_kernels": {"bf16": {"cpu_moe_gbs": 0.0, "pcie_gather_gbs": 10.0}}}
    assert BP.load_hybrid_fetch_fraction("bf16", path=_write(tmp_path, zero)) is None
    big = {"gpu": {"name": "Test GPU"}, "dtype_kernels": {"bf16": {"cpu_moe_gbs": 5.0, "pcie_gather_gbs": 10.0}}}
    assert BP.load_hybrid_fetch_fraction("bf16", path=_write(tmp_path, big)) == 1.0  # clamped


def test_fetch_fraction_none_without_profile(tmp_path, monkeypatch):
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    monkeypatch.setattr(BP, "gpu_identity", lambda: (None, None))
    assert BP.load_hybrid_fetch_fraction("bf16") is None


def test_env_var_selects_the_profile(tmp_path, monkeypatch):
    monkeypatch.setattr(BP, "gpu_identity", lambda: ("Test GPU", "uuid-9"))
    monkeypatch.setenv(BP.ENV_PROFILE_PATH, _write(tmp_path, _hybrid_profile()))
    assert BP.load_backend_recommendation("bf16") == "hybrid"
    assert BP.load_hybrid_fetch_fraction("bf16") == pytest.approx(8 / 28)


def test_per_device_file_found_by_uuid(tmp_path, monkeypatch):
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    monkeypatch.setattr(BP, "gpu_identity", lambda: ("Test GPU", "uuid-0"))
    p = BP.default_profile_path("uuid-0")
    os.makedirs(os.path.dirname(p))
    with open(p, "w") as f:
        json.dump(_hybrid_profile(), f)
    assert BP.load_backend_recommendation("bf16") == "hybrid"


def test_resolve_backend(tmp_path, monkeypatch):
    monkeypatch.setattr(BP, "is_gpu_available", lambda: True)
    monkeypatch.setattr(BP, "gpu_identity", lambda: ("Test GPU", "uuid-0"))
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    (tmp_path / "freetoken").mkdir()
    assert BP.resolve_backend("auto", is_moe=True, quant_format="bf16") == "offload"  # no profile
    assert BP.resolve_backend("auto", is_moe=False) == "fused"
    assert BP.resolve_backend("cpu", is_moe=True, quant_format="bf16") == "cpu"
    monkeypatch.setenv(BP.ENV_PROFILE_PATH, _write(tmp_path, _hybrid_profile()))
    assert BP.resolve_backend("auto", is_moe=True, quant_format="bf16") == "hybrid"
    monkeypatch.setattr(BP, "is_gpu_available", lambda: False)
    assert BP.resolve_backend("auto", is_moe=True, quant_format="bf16") == "fused"


def test_quant_format_for_dtype():
    import torch

    assert BP.quant_format_for_dtype(torch.bfloat16) == "bf16"
    assert BP.quant_format_for_dtype("fp8") == "fp8_block"
    assert BP.quant_format_for_dtype("mxfp4_triton") == "mxfp4"
    assert BP.quant_format_for_dtype("gptq_int4") == "gptq_int4"
    assert BP.quant_format_for_dtype(None) is None and BP.quant_format_for_dtype("") is None


# ---- the writer's host-side parts -------------------------------------------------------


def test_verdict_and_fraction():
    assert BW._recommend(10.0, 25.0) == "hybrid" and BW._recommend(10.0, 20.0) == "offload"
    assert BW._recommend(None, 5.0) == "offload" and BW._recommend(0.0, 5.0) == "offload"
    assert BW._fetch_fraction(8.0, 24.0, 1.0, 1.0) == pytest.approx(0.25)  # overlapped pair first
    assert BW._fetch_fraction(None, None, 10.0, 30.0) == pytest.approx(0.25)
    assert BW._fetch_fraction(None, None, None, 30.0) == 0.0


@pytest.mark.parametrize("name", ["c1_int8", "c2_gptq", "c3_fp8", "c4_mxfp4"])
def test_synthetic_bank_bytes_are_the_configs_expert_bytes(name):
    cfg = S.CONFIGS[name]
    bank = BW.synthetic_banks(cfg.fmt, 2, cfg.I, cfg.H, distinct=1, bias=cfg.expert_bias)
    assert BW.expert_bytes(bank) == cfg.bytes_per_expert
    for t in bank.values():
        assert t.shape[0] == 2 and t[0].data_ptr() != t[1].data_ptr()


@pytest.mark.parametrize("fmt", BW.FORMATS)
def test_cpu_half_bandwidth_runs_on_the_host(fmt):
    bank = BW.synthetic_banks(fmt, 8, 256, 512, distinct=2)
    gbs = BW.bench_cpu_moe(fmt, bank, 8, 256, 512, iters=2, threads=2)
    assert gbs > 0.01


def test_workload_resolution(tmp_path):
    args = BW.parse_argv([])
    assert BW.resolve_workload(args) == (64, 768, 2048, ["bf16"])
    args = BW.parse_argv(["--dtype", "fp8,gptq_int4", "--experts", "8", "--intermediate", "256", "--hidden", "512"])
    assert BW.resolve_workload(args) == (8, 256, 512, ["fp8_block", "gptq_int4"])
    assert BW.resolve_workload(BW.parse_argv(["--dtype", "all"]))[3] == list(BW.FORMATS)
    with pytest.raises(ValueError, match="unknown expert format"):
        BW.resolve_workload(BW.parse_argv(["--dtype", "nvfp4"]))
    cfg = {"num_hidden_layers": 4, "num_experts": 128, "hidden_size": 2048, "moe_intermediate_size": 768,
           "quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 128}}
    (tmp_path / "config.json").write_text(json.dumps({"text_config": cfg}))
    assert BW.resolve_workload(BW.parse_argv(["--model", str(tmp_path)])) == (128, 768, 2048, ["gptq_int4"])
    assert BW.resolve_workload(BW.parse_argv(["--model", str(tmp_path), "--experts", "16"]))[0] == 16


def test_main_without_a_gpu_exits_1(monkeypatch, capsys):
    monkeypatch.setattr(BP, "is_gpu_available", lambda: False)
    assert BW.main(["--dtype", "bf16"]) == 1
    assert "needs a ROCm GPU" in capsys.readouterr().err
