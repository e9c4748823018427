"""The process-wide host thread pool that packing runs on (csrc/par.h): a stress
check built with g++'s thread sanitizer and run here on the CPU. Several owners
at once, nested loops, exceptions and the one-thread budget, every result
checked (tests/native/host_pool_check.cpp)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "host_pool_check.cpp")
INC = os.path.join(ROOT, "war-chest-bot-9000-_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_pool_under_the_thread_sanitizer(tmp_path):
    exe = str(tmp_path / "host_pool_check")
    build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=thread", "-I", INC, SRC, "-o", exe,
                            "-lpthread"], capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-2000:]
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "0 wrong results, 480 exceptions delivered" in run.stdout
