"""Sanitizer runs of the library's host-only code -- the slot-pool LRU
(csrc/ftm_offload.cpp) and the CPU expert kernel of the hybrid split with its
async worker (csrc/ftm_cpu.cpp) -- driven by tests/host_sanitize_driver.cpp:
AddressSanitizer + UndefinedBehaviorSanitizer over random shapes, routings,
corrupt caller state and argument errors, and ThreadSanitizer over several
host threads submitting to and waiting on the worker beside synchronous
multi-threaded calls (the reference documents a constructor-order race in
its AsyncWorker, python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:676-697).
g++ builds the sanitized copies (host code only; no GPU code is compiled with
a sanitizer), with the sanitizer runtimes linked statically so the
executables need nothing from the environment's library search order."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "freetoken-intel_amd", "csrc")


def _build(tmp_path, name, sanitize):
    exe = str(tmp_path / name)
    static = ["-static-libasan", "-static-libubsan"] if "address" in sanitize else ["-static-libtsan"]
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-pthread", f"-fsanitize={sanitize}",
           "-fno-sanitize-recover=all", *static, "-I", os.path.join(ROOT, "include"),
           os.path.join(HERE, "host_sanitize_driver.cpp"), os.path.join(CSRC, "ftm_offload.cpp"),
           os.path.join(CSRC, "ftm_cpu.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    return exe


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_code_under_asan_and_ubsan(tmp_path):
    exe = _build(tmp_path, "host_asan", "address,undefined")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "host sanitize driver: ok" in r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_async_worker_under_tsan(tmp_path):
    exe = _build(tmp_path, "host_tsan", "thread")
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1:second_deadlock_stack=1")
    r = subprocess.run([exe, "threads"], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-6000:]
    assert "host sanitize driver (threads): ok" in r.stdout
    assert "WARNING: ThreadSanitizer" not in r.stderr
