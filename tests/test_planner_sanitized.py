"""The host planner and the host driver (page allocator, step metadata) built
with AddressSanitizer and UndefinedBehaviorSanitizer (g++, host code only):
random batches and serving steps must plan into lists whose every index
stays in bounds and whose pieces cover every (rows, kv head) token range
exactly once, and corrupted metadata must be refused
(tests/cpp/planner_check.cpp)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_planner_under_sanitizers(tmp_path):
    exe = tmp_path / "planner_check"
    build = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-fno-omit-frame-pointer", "-I" + os.path.join(ROOT, "include"),
             "-I" + os.path.join(ROOT, "flashengine.cpp_amd", "csrc"),
             os.path.join(ROOT, "tests", "cpp", "planner_check.cpp"),
             os.path.join(ROOT, "flashengine.cpp_amd", "csrc", "planner.cpp"),
             os.path.join(ROOT, "flashengine.cpp_amd", "csrc", "driver.cpp"), "-o", str(exe)]
    subprocess.run(build, check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), "1500", "600"], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert lines[-1].startswith("ok: ") and any(line.startswith("prefix cache: ") for line in lines)
