"""The library's host-only C++ (tokenizer.cpp with its worker threads,
safetensors.cpp fed truncated and corrupted files, embed.cpp, and
host_sched.cpp: options, pass planning, the workspace free list and the
serving batcher's queue under concurrent clients) built with
g++ under AddressSanitizer + UndefinedBehaviorSanitizer and under
ThreadSanitizer, and run on the CPU by tests/sanitize/host_check.cpp (no
GPU: the model entry points those files call are stubbed there)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "indecis_amd", "csrc")
SOURCES = [os.path.join(CSRC, f) for f in ("tokenizer.cpp", "safetensors.cpp", "embed.cpp", "host_sched.cpp")]
DRIVER = os.path.join(ROOT, "tests", "sanitize", "host_check.cpp")
TOKENIZER = os.path.join(ROOT, "tests", "golden", "tokenizer", "tokenizer.json")
SANITIZERS = {
    "address": ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"],
    "thread": ["-fsanitize=thread"],
}


@pytest.mark.parametrize("kind", sorted(SANITIZERS))
def test_host_code_under_sanitizer(kind, tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / f"host_check_{kind}"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-pthread", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           *SANITIZERS[kind], DRIVER, *SOURCES, "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               TSAN_OPTIONS="halt_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), TOKENIZER, str(tmp_path)], capture_output=True, text=True, env=env,
                       timeout=600)
    report = r.stderr[-6000:]
    assert r.returncode == 0, report
    assert "host_check: ok" in r.stderr
    assert "Sanitizer" not in r.stderr, report
