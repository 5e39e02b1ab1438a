"""The host-table path's thread pool (lanternl_amd/csrc/lhip_pool.h), built on
its own with g++ and stressed on the CPU: every part of every run exactly once,
run() returning only after all parts returned, workers falling asleep and
waking between runs, stop and restart.  Once plain, once under
ThreadSanitizer (host code only)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "host_pool_check.cpp")


def _build_and_run(tmp_path, flags, iters):
    if not shutil.which("g++"):
        pytest.skip("g++ not found")
    exe = str(tmp_path / "host_pool_check")
    subprocess.run(["g++", "-std=c++17", "-O2", "-g", "-pthread", *flags, SRC, "-o", exe], check=True,
                   capture_output=True, text=True)
    r = subprocess.run([exe, str(iters)], capture_output=True, text=True, timeout=240)
    return r


def test_pool_runs_every_part_once(tmp_path):
    r = _build_and_run(tmp_path, [], 20000)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr


def test_pool_is_race_free_under_tsan(tmp_path):
    r = _build_and_run(tmp_path, ["-fsanitize=thread"], 3000)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
