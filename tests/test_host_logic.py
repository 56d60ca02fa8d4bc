"""Host-side logic of the library checked on the CPU, built with
AddressSanitizer and UndefinedBehaviorSanitizer (host code only; no GPU).

- The device-pointer scratch pool's growth rule (csrc/scratch_pool.h): a
  buffer handed to a stream is never freed or shared while the pool lives.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _run(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_scratch_pool_growth_rule_under_asan(tmp_path):
    exe = str(tmp_path / "scratch_pool_test")
    subprocess.run(["g++", "-std=c++17", *SAN, "-pthread", os.path.join(CPP, "scratch_pool_test.cpp"),
                    "-o", exe], check=True, timeout=300)
    assert "scratch pool ok" in _run(exe)
