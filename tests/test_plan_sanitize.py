"""The host-side planning code (csrc/host_plan.h: argument checks, workspace
layout, worker grid, launch shape) built for the CPU with g++ and the
address and undefined-behaviour sanitizers, then swept over extreme batch,
head, split, worker and capacity values (tests/plan_sanitize.cpp): no signed
overflow, no wrapped size, and the invariants the kernels rely on."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_planning_under_sanitizers(tmp_path):
    exe = tmp_path / "plan_sanitize"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "triton-mla_amd", "csrc"), os.path.join(HERE, "plan_sanitize.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, (run.stdout + run.stderr)[-3000:]
    assert run.stdout.startswith("ok ")
