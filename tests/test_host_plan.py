"""Host logic under the address and undefined-behaviour sanitizers (CPU).

Builds two native checks with g++ -fsanitize=address,undefined and runs them:
  - tests/native/plan_check.cpp over aegean-tge_amd/host/plan.cpp: random
    step plans (decode and block-prefill work lists cover every page once,
    split slots and reduction records agree), rejected descriptions, and
    staged uploads that survive injected allocation failures;
  - tests/native/driver_host_check.cpp over aegean-tge_amd/host/qwen2_kv.cpp
    with a stand-in for the device entry points: transactional begin under
    injected plan and copy failures, exact token-by-token prefix matching,
    and a random flow whose attaches are checked against page contents.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FLAGS = ["-std=c++20", "-O1", "-g", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=all", "-Wall", "-Wextra", "-Werror",
         "-I" + os.path.join(ROOT, "include")]


def build_and_run(tmp_path, name, sources):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    exe = str(tmp_path / name)
    cmd = ["g++", *FLAGS, *[os.path.join(ROOT, s) for s in sources], "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    return r.stdout


def test_planner_under_sanitizers(tmp_path):
    out = build_and_run(tmp_path, "plan_check",
                        ["aegean-tge_amd/host/plan.cpp", "tests/native/plan_check.cpp"])
    assert "plan_check ok" in out


def test_driver_bookkeeping_under_sanitizers(tmp_path):
    out = build_and_run(tmp_path, "driver_host_check",
                        ["aegean-tge_amd/host/qwen2_kv.cpp", "tests/native/driver_host_check.cpp"])
    assert "driver_host_check ok" in out
