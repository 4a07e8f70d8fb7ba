"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

host_rules.cpp (packers, unpackers, argument validators) is plain C++; this
test builds it with g++ -fsanitize=address,undefined together with
tests/asan/host_rules_driver.cpp and runs the pack round trips (on exactly
sized heap buffers, so an index past either buffer is an ASan report) and the
rejection cases.  A sanitizer report fails the run (halt_on_error)."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_rules_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "host_rules_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", f"-I{REPO / 'include'}", f"-I{REPO / 'leanstack_amd' / 'csrc'}",
           str(REPO / "leanstack_amd" / "csrc" / "host_rules.cpp"), str(REPO / "tests" / "asan" / "host_rules_driver.cpp"),
           "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert run.returncode == 0 and run.stdout.strip().endswith("ok"), run.stdout + run.stderr
