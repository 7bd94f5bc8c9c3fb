"""CPU tests of the context's host worker pool (cuda-zkml_amd/csrc/worker_pool.hpp).

zk_prove runs its MSM jobs and the three-set MSM's per-set window
combinations on these workers, and a job waits on its own sub-tasks, so the
pool must run every task exactly once and never leave a waiter on a task no
worker will take.  tests/native/worker_pool_check.cpp drives it with flat,
nested and multi-submitter loads on pools of 1, 2 and 5 workers, spinning and
sleeping, and is also built under ThreadSanitizer (host code only) to catch
data races in the hand-off.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cuda-zkml_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "native", "worker_pool_check.cpp")


def build_and_run(tmp_path, extra):
    exe = tmp_path / "worker_pool_check"
    subprocess.run(["g++", "-O2", "-g", "-std=c++17", "-pthread", *extra, "-I", CSRC, SRC, "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "worker pool ok" in r.stdout
    return r


def test_worker_pool(tmp_path):
    build_and_run(tmp_path, [])


def test_worker_pool_thread_sanitizer(tmp_path):
    probe = subprocess.run(["g++", "-fsanitize=thread", "-x", "c++", "-", "-o", str(tmp_path / "probe")],
                           input="int main(){}", text=True, capture_output=True)
    if probe.returncode != 0:
        pytest.skip("ThreadSanitizer runtime not available to g++ here")
    r = build_and_run(tmp_path, ["-fsanitize=thread"])
    assert "WARNING: ThreadSanitizer" not in r.stderr, r.stderr
