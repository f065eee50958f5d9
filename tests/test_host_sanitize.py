"""AddressSanitizer + UndefinedBehaviorSanitizer run of the library's
host-only code -- the slot-pool LRU (csrc/ftm_offload.cpp) and the CPU expert
kernel of the hybrid split (csrc/ftm_cpu.cpp) -- driven by
tests/host_sanitize_driver.cpp with random shapes, routings, corrupt caller
state and argument errors.  g++ builds the sanitized copy (host code only;
no GPU code is compiled with a sanitizer)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "freetoken-intel_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_code_under_asan_and_ubsan(tmp_path):
    exe = str(tmp_path / "host_sanitize")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-pthread",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "include"),
           os.path.join(HERE, "host_sanitize_driver.cpp"), os.path.join(CSRC, "ftm_offload.cpp"),
           os.path.join(CSRC, "ftm_cpu.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "host sanitize driver: ok" in r.stdout
