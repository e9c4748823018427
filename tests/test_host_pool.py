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


def test_packing_in_a_child_forked_after_the_pool_ran():
    """A child process forked after the library's host pool has run (as
    fork-started worker processes are) packs waves exactly as its parent does:
    no worker holds the pool's lock across the fork, and the child runs its
    loops on the calling thread. The child gets 60 s; a hang fails the test."""
    import time

    import warchest_wave as ww
    import workloads as W

    import threading

    jobs = W.jobs("wave64", trees=8)
    want = ww.Wave(jobs).digest()  # the pool is up and has run
    busy, stop = [], threading.Event()

    def keep_packing():  # the pool's workers busy at the fork
        while not stop.is_set():
            busy.append(ww.Wave(jobs).digest() == want)

    t = threading.Thread(target=keep_packing, daemon=True)
    t.start()
    try:
        while not busy:
            time.sleep(0.01)
        pid = os.fork()
        if pid == 0:  # the child: exit status 0 only if its pack matches
            code = 3
            try:
                code = 0 if ww.Wave(jobs).digest() == want else 2
            finally:
                os._exit(code)
        deadline = time.time() + 60
        while True:
            done, status = os.waitpid(pid, os.WNOHANG)
            if done:
                break
            if time.time() > deadline:
                os.kill(pid, 9)
                os.waitpid(pid, 0)
                pytest.fail("the forked child did not finish packing within 60 s")
            time.sleep(0.05)
    finally:
        stop.set()
        t.join()
    assert all(busy)
    assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0, status
